"""Parity of libhq.so's HIP kernels with the oracle (the reference's arithmetic), through the C-ABI, on cuda:0.

Integers and bytes exact, every float32 output to the bit (the kernels keep the reference's float32 order), and
nothing written outside the rows / tokens of a call (outputs start at -7, as tests/int8-check.ts:176-181 checks).
The cases are the reference tests' (tests/int8-check.ts, tests/ternary-check.ts: their group counts, row ranges,
token counts, int8 ends, zero and subnormal scales, the largest sums), the order-revealing inputs of
test_oracle.py; test_gpu_shapes.py holds the benchmark configs' shapes at full size.
"""
import numpy as np
import pytest

import models
from gpu_util import Arena, first_difference, same_bits
from models import F
from streams import LCG, pack6, pack_binary, pack_ternary, scale_rule
from test_oracle import quantize_cases

pytestmark = pytest.mark.gpu

ROWS = 13
RANGES = [(0, ROWS), (0, 1), (0, 3), (ROWS - 1, ROWS), (1, 6), (3, 8), (5, 5), (4, 12)]
GROUPS = [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 13, 80, 81]


@pytest.fixture(scope="module")
def k(pkg):
    import torch
    assert torch.cuda.is_available(), "the GPU tests need a GPU"
    return pkg.load_kernels()


@pytest.fixture(scope="module")
def arena():
    return Arena(1 << 30)


@pytest.fixture(autouse=True)
def fresh(arena):
    arena.reset()
    yield


def expect_range(full, r0, r1, rows=ROWS):
    want = np.full(rows + 1, F(-7), F)
    want[r0:r1] = full[r0:r1]
    return want


# ---- activations and corrections ------------------------------------------------------------------------------
@pytest.mark.parametrize("bias", [0, 64])
def test_quantize_x(k, arena, oracle, bias):
    x = quantize_cases()
    rng = np.random.default_rng(bias)
    x = np.concatenate([x, rng.standard_normal(32 * 50).astype(F) * 3])
    n = x.size
    ax = arena.put(x)
    xq = arena.alloc(n + 64, fill=np.full(n + 64, 0xAA, np.uint8))
    xs = arena.alloc(4 * (n // 32) + 64, fill=np.full(n // 8 + 64, 0xAA, np.uint8))
    k.quantize_x(xq, xs, ax, n, bias)
    want_q, want_s = oracle.quantize_x(x, bias)
    got_q = arena.get(xq, np.uint8, n + 64)
    got_s = arena.get(xs, F, n // 32 + 16)
    assert np.array_equal(got_q[:n], want_q)
    assert same_bits(got_s[: n // 32], want_s)
    assert np.all(got_q[n:] == 0xAA) and np.all(got_s[n // 32:].view(np.uint32) == 0xAAAAAAAA)


def test_quantize_x_nan_groups(k, arena, oracle):
    x = np.ones(96, F)
    x[0] = np.nan
    x[32 + 5] = np.nan
    x[32 + 1] = F(2.0)
    x[64 + 3] = np.inf
    xq, xs = arena.alloc(96), arena.alloc(12)
    k.quantize_x(xq, xs, arena.put(x), 96, 64)
    want_q, want_s = oracle.quantize_x(x, 64)
    assert np.array_equal(arena.get(xq, np.uint8, 96), want_q)
    got_s = arena.get(xs, F, 3)
    assert np.array_equal(np.isnan(got_s), np.isnan(want_s))
    assert got_s[1] == want_s[1]


@pytest.mark.parametrize("n,count,frame", [(1024, 7, 2048), (4608, 3, 5248), (14336, 4, 16128)])
def test_quantize_x_batch(pkg, arena, oracle, n, count, frame):
    """tokens of a batch: each token's group index taken apart as token and group (group counts 32, 144, 448)"""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((count, n)).astype(F)
    ax = arena.put(x)
    xq = arena.alloc(count * frame)
    L = pkg.library()
    assert L.hq_quantize_x_batch(xq, xq + n, ax, n, 64, count, frame, 4 * n, None) == 0
    for t in range(count):
        want_q, want_s = oracle.quantize_x(x[t], 64)
        assert np.array_equal(arena.get(xq + t * frame, np.uint8, n), want_q)
        assert same_bits(arena.get(xq + t * frame + n, F, n // 32), want_s)


def test_int8_and_six_sums(k, arena, oracle):
    rng = np.random.default_rng(3)
    w = rng.integers(-128, 128, 32 * 777).astype(np.int8)
    w[:32], w[32:64] = 127, -128
    out = arena.alloc(4 * 780, fill=np.full(780, -7, np.int32))
    k.int8_sums(out, arena.put(w), 777)
    got = arena.get(out, np.int32, 778)
    assert np.array_equal(got[:777], oracle.int8_sums(w)) and got[777] == -7
    v = (4 * rng.integers(-32, 32, 32 * 333)).astype(np.int8)
    v[:32], v[32:64] = 124, -128
    packed = pack6(v)
    out6 = arena.alloc(4 * 340, fill=np.full(340, -7, np.int32))
    k.six_sums(out6, arena.put(packed), 333)
    got6 = arena.get(out6, np.int32, 334)
    assert np.array_equal(got6[:333], oracle.six_sums(packed)) and got6[333] == -7


@pytest.mark.parametrize("n", [128, 256, 384, 640, 1152, 17408])
def test_interleave(k, arena, oracle, n):
    rng = LCG(231 + n)
    a = np.array([(rng.next() & 255) - 128 for _ in range(n)], np.int8)
    a[:32], a[32:64] = 127, -128
    xs = (np.arange(n // 32) + 0.5).astype(F)
    xq = arena.put(np.concatenate([a, np.full(64, 55, np.int8)]))
    area = arena.put(np.concatenate([xs, np.full(n // 32 + 2, -7, np.int32).view(F)]))
    k.interleave(xq, area, n)
    want_bytes, want_area = oracle.interleave(a, xs)
    assert np.array_equal(arena.get(xq, np.int8, n + 64), np.concatenate([want_bytes, np.full(64, 55, np.int8)]))
    got_area = arena.get(area, F, 2 * (n // 32) + 2)
    assert same_bits(got_area[: 2 * (n // 32)], want_area)
    assert np.all(got_area[2 * (n // 32):].view(np.int32) == -7)


def test_interleave_batch(pkg, arena, oracle):
    rng = np.random.default_rng(5)
    n, count, frame = 5120, 5, 8192
    a = rng.integers(-128, 128, (count, n)).astype(np.int8)
    xs = rng.random((count, n // 32)).astype(F)
    buf = arena.alloc(count * frame)
    for t in range(count):
        arena.write(buf + t * frame, a[t])
        arena.write(buf + t * frame + n, xs[t])
    assert pkg.library().hq_interleave_batch(buf, buf + n, n, count, frame, None) == 0
    for t in range(count):
        want_bytes, want_area = oracle.interleave(a[t], xs[t])
        assert np.array_equal(arena.get(buf + t * frame, np.int8, n), want_bytes)
        assert same_bits(arena.get(buf + t * frame + n, F, 2 * (n // 32)), want_area)


# ---- int8 / int6 token kernels --------------------------------------------------------------------------------
def int8_case(ng, tokens=9):
    """tests/int8-check.ts:129-171: int8 weights (-128 too, rows 0/1 at the ends, row 2 alternating), int6 ones,
    scales of every size, activations: token 0 all 127, 1 all 0, 2 alternating, 3 quantize_x of floats, others
    random (relaxed, 0..127); and the plain form's -127..127 patterns."""
    rng = LCG(644 + 7 * ng)
    n = ng * 32
    w8 = np.array([(rng.next() & 255) - 128 for _ in range(ROWS * n)], np.int8)
    v6 = np.array([4 * ((rng.next() & 63) - 32) for _ in range(ROWS * n)], np.int8)
    w8[:n], w8[n:2 * n] = 127, -128
    v6[:n], v6[n:2 * n] = 124, -128
    w8[2 * n:3 * n] = np.where(np.arange(n) & 1, 127, -128)
    v6[2 * n:3 * n] = np.where(np.arange(n) & 1, 124, -128)
    ws = np.array([scale_rule(rng, i) for i in range(ROWS * ng)], F)
    xf = np.array([F(((rng.next() % 2001) - 1000) * 1e-3 * (1 + j % 5)) for j in range(n)], F)
    relaxed, plain = [], []
    for t in range(tokens):
        s = np.array([scale_rule(rng, g + t) for g in range(ng)], F)
        if t == 3:  # quantize_x of the floats xf, at the form's bias
            relaxed.append((None, None))
            plain.append((None, None))
            continue
        if t == 0:
            u, i8 = np.full(n, 127, np.uint8), np.full(n, 127, np.int8)
        elif t == 1:
            u, i8 = np.zeros(n, np.uint8), np.full(n, -127, np.int8)
        elif t == 2:
            u = np.where(np.arange(n) & 1, 127, 0).astype(np.uint8)
            i8 = np.where(np.arange(n) & 1, 127, -127).astype(np.int8)
        else:
            u = np.array([rng.next() & 127 for _ in range(n)], np.uint8)
            i8 = np.array([(rng.next() % 255) - 127 for _ in range(n)], np.int8)
        relaxed.append((u, s))
        plain.append((i8, s))
    return n, w8, v6, ws, xf, relaxed, plain


def quantized_tokens(oracle, xf, toks, bias):
    out = []
    for (q, s) in toks:
        if q is None:
            q, s = oracle.quantize_x(xf, bias)
            if bias == 0:
                q = q.view(np.int8)
        out.append((q, s))
    return out


def run_token_kernel(k, arena, name, n, wq_addr, ws_addr, wc_addr, q, s, r0, r1):
    xq = arena.put(q)
    xs = arena.put(s)
    out = arena.alloc(4 * (ROWS + 1), fill=np.full(ROWS + 1, -7, F))
    fn = getattr(k, name)
    if name in ("matmul_q8r", "matmul_q6r"):
        fn(out, xq, xs, wq_addr, ws_addr, wc_addr, n, r0, r1)
    else:
        fn(out, xq, xs, wq_addr, ws_addr, n, r0, r1)
    return arena.get(out, F, ROWS + 1)


@pytest.mark.parametrize("ng", GROUPS)
@pytest.mark.parametrize("form", ["matmul_q8r", "matmul_q8r_derived", "matmul_q6r", "matmul_q6r_derived", "matmul_q8",
                                  "matmul_q6"])
def test_token_kernels(k, arena, oracle, ng, form):
    n, w8, v6, ws, xf, relaxed, plain = int8_case(ng)
    six = form in ("matmul_q6r", "matmul_q6r_derived", "matmul_q6")
    wbytes = pack6(v6) if six else w8
    wq = arena.put(wbytes)
    wsa = arena.put(ws)
    is_relaxed = form.startswith("matmul_q8r") or form.startswith("matmul_q6r")
    toks = quantized_tokens(oracle, xf, relaxed if is_relaxed else plain, 64 if is_relaxed else 0)
    wc = (oracle.six_sums(wbytes) if six else oracle.int8_sums(w8)) if is_relaxed else None
    wca = arena.put(wc) if form in ("matmul_q8r", "matmul_q6r") else 0  # the _derived forms pass wc = NULL
    name = form[:-len("_derived")] if form.endswith("_derived") else form
    for t, (q, s) in enumerate(toks):
        if is_relaxed:
            full = (oracle.matmul_q6r if six else oracle.matmul_q8r)(q, s, wbytes, ws, wc, n)
        else:
            full = (oracle.matmul_q6 if six else oracle.matmul_q8)(q, s, wbytes, ws, n)
        for r0, r1 in RANGES:
            got = run_token_kernel(k, arena, name, n, wq, wsa, wca, q, s, r0, r1)
            want = expect_range(full, r0, r1)
            assert same_bits(got, want), f"{form} ng {ng} token {t} rows {r0}..{r1}: {first_difference(got, want)}"


# ---- the tile: every (row, token) is matmul_q8r's number ------------------------------------------------------
def tile_inputs(oracle, rng, n, count, frame, rows):
    x = rng.standard_normal((count, n)).astype(F)
    x[0, :32] = 0  # a group of zeros: scale 0
    q = np.zeros((count, frame), np.uint8)
    for t in range(count):
        qq, ss = oracle.quantize_x(x[t], 64)
        q[t, :n] = qq
        q[t, n:n + 4 * (n // 32)] = ss.view(np.uint8)
    return q


@pytest.mark.parametrize("count", [1, 2, 3, 4, 5, 7, 8, 9, 16, 17, 33, 64, 65, 100])
@pytest.mark.parametrize("ng", [1, 3, 4, 9, 13, 80])
def test_q8r_tile(k, arena, oracle, count, ng):
    rng = np.random.default_rng(1000 * ng + count)
    n = 32 * ng
    rows = 70
    frame = ((n + 4 * ng + 15) // 16) * 16
    os_ = 4 * (rows + 3)
    w = rng.integers(-128, 128, rows * n).astype(np.int8)
    ws = (rng.random(rows * ng) * 1e-3).astype(F)
    ws[::11] = F(2.0 ** -130)
    ws[5::13] = 0
    wc = oracle.int8_sums(w)
    # a caller's own corrections: int8_sums' values with a few groups moved (the kernels add whatever wc holds)
    moved = wc.copy()
    moved[rng.integers(0, rows * ng, 3)] += np.array([1, -5000, 77], np.int32)
    q = tile_inputs(oracle, rng, n, count, frame, rows)
    wq, wsa, xq = arena.put(w), arena.put(ws), arena.put(q)
    for form, corrections in (("int8_sums", wc), ("derived", None), ("moved", moved)):
        wca = 0 if corrections is None else arena.put(corrections)
        for r0, r1 in [(0, rows), (3, 64 + 3), (5, 6)]:
            out = arena.alloc(os_ * count, fill=np.full(os_ * count // 4, -7, F))
            k.matmul_q8r_tile(out, xq, xq + n, wq, wsa, wca, n, r0, r1, count, os_, frame)
            got = arena.get(out, F, os_ * count // 4).reshape(count, -1)
            for t in range(count):
                full = oracle.matmul_q8r(q[t, :n], q[t, n:n + 4 * ng].view(F), w, ws,
                                         wc if corrections is None else corrections, n)
                want = np.full(os_ // 4, F(-7), F)
                want[r0:r1] = full[r0:r1]
                assert same_bits(got[t], want), f"count {count} ng {ng} rows {r0}..{r1} token {t} wc {form}: " \
                                                f"{first_difference(got[t], want)}"


@pytest.mark.parametrize("count", [2, 3, 4])
@pytest.mark.parametrize("packing", ["int8", "int6"])
@pytest.mark.parametrize("ng", [544, 1152])
def test_relaxed_tokens_long_rows(pkg, k, arena, oracle, count, packing, ng):
    """2..4 tokens of long rows: 17408 values, whose activations (39-78 KB) are staged in LDS, and 36864, whose
    activations (more than 80 KB for two tokens) are read through the caches; rows cut, the corrections given,
    derived and moved"""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(31 + count + ng)
    rows = 37
    n = 32 * ng
    frame = ((n + 4 * ng + 15) // 16) * 16
    assert (count * (n + 4 * ng) > 80 * 1024) == (ng == 1152)
    if packing == "int8":
        w = rng.integers(-128, 128, rows * n).astype(np.int8)
        wbytes, sums = w, oracle.int8_sums(w)
    else:
        wbytes = pack6((4 * rng.integers(-32, 32, rows * n)).astype(np.int8))
        sums = oracle.six_sums(wbytes)
    ws = (rng.random(rows * ng) * 1e-3).astype(F)
    moved = sums.copy()
    moved[rng.integers(0, rows * ng, 3)] += np.array([1, -5000, 77], np.int32)
    q = tile_inputs(oracle, rng, n, count, frame, rows)
    wq, wsa, xq = arena.put(wbytes, align=256), arena.put(ws), arena.put(q)
    kind = "matmul_q8r" if packing == "int8" else "matmul_q6r"
    product = oracle.matmul_q8r if packing == "int8" else oracle.matmul_q6r
    forms = (("sums", sums), ("derived", None), ("moved", moved))
    for form, corrections in forms:
        wca = 0 if corrections is None else arena.put(corrections)
        # int8 through the drop-in tile (rows cut at both ends), int6 through a phase (a job's rows start at 0)
        for r0, r1 in ([(0, rows), (3, 20)] if packing == "int8" else [(0, rows), (0, 20)]):
            out = arena.alloc(4 * rows * count, fill=np.full(rows * count, -7, F))
            if packing == "int8":
                k.matmul_q8r_tile(out, xq, xq + n, wq, wsa, wca, n, r0, r1, count, 4 * rows, frame)
            else:
                job = jobs.job(kind, out, xq, xq + n, wq, wsa, wca, n, rows=r1, count=count, os=4 * rows, as_=frame,
                               bs=frame)
                assert jobs.phase(pkg.library(), [job]) == 0, pkg.library().hq_last_error_message()
            got = arena.get(out, F, rows * count).reshape(count, rows)
            for t in range(count):
                full = product(q[t, :n], q[t, n:n + 4 * ng].view(F), wbytes, ws,
                               sums if corrections is None else corrections, n)
                want = np.full(rows, F(-7), F)
                want[r0:r1] = full[r0:r1]
                assert same_bits(got[t], want), f"{packing} count {count} rows {r0}..{r1} token {t} wc {form}: " \
                                                f"{first_difference(got[t], want)}"


@pytest.mark.parametrize("count,ng,packing", [(1, 128, "int8"), (1, 256, "int8"), (1, 320, "int8"), (1, 448, "int8"),
                                               (2, 259, "int8"), (3, 259, "int8"), (4, 259, "int8"), (2, 259, "int6"),
                                               (3, 259, "int6")])
def test_relaxed_wide_rows(pkg, k, arena, oracle, count, ng, packing):
    """The launches whose relaxed rows are 32 lanes (one int8 token on rows of 4096 or 8192 values, and of 10240 or
    14336 in chunks of two steps; 2..4 tokens on rows past 8192 — 2 and 3 tokens of 8288 values staged in LDS, 4 read
    through the caches, with 3 groups past the fours): rows cut inside the 4-row blocks at both ends, the corrections
    given, derived and moved"""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(71 + count + ng)
    rows = 37
    n = 32 * ng
    frame = ((n + 4 * ng + 15) // 16) * 16
    if packing == "int8":
        w = rng.integers(-128, 128, rows * n).astype(np.int8)
        wbytes, sums = w, oracle.int8_sums(w)
    else:
        wbytes = pack6((4 * rng.integers(-32, 32, rows * n)).astype(np.int8))
        sums = oracle.six_sums(wbytes)
    ws = (rng.random(rows * ng) * 1e-3).astype(F)
    moved = sums.copy()
    moved[rng.integers(0, rows * ng, 3)] += np.array([1, -5000, 77], np.int32)
    q = tile_inputs(oracle, rng, n, count, frame, rows)
    wq, wsa, xq = arena.put(wbytes, align=256), arena.put(ws), arena.put(q)
    kind = "matmul_q8r" if packing == "int8" else "matmul_q6r"
    product = oracle.matmul_q8r if packing == "int8" else oracle.matmul_q6r
    for form, corrections in (("sums", sums), ("derived", None), ("moved", moved)):
        wca = 0 if corrections is None else arena.put(corrections)
        for r0, r1 in ([(0, rows), (3, 34)] if packing == "int8" else [(0, rows), (0, 34)]):
            out = arena.alloc(4 * rows * count, fill=np.full(rows * count, -7, F))
            if packing == "int8":
                k.matmul_q8r_tile(out, xq, xq + n, wq, wsa, wca, n, r0, r1, count, 4 * rows, frame)
            else:
                job = jobs.job(kind, out, xq, xq + n, wq, wsa, wca, n, rows=r1, count=count, os=4 * rows, as_=frame,
                               bs=frame)
                assert jobs.phase(pkg.library(), [job]) == 0, pkg.library().hq_last_error_message()
            got = arena.get(out, F, rows * count).reshape(count, rows)
            for t in range(count):
                full = product(q[t, :n], q[t, n:n + 4 * ng].view(F), wbytes, ws,
                               sums if corrections is None else corrections, n)
                want = np.full(rows, F(-7), F)
                want[r0:r1] = full[r0:r1]
                assert same_bits(got[t], want), f"{packing} count {count} ng {ng} rows {r0}..{r1} token {t} " \
                                                f"wc {form}: {first_difference(got[t], want)}"


@pytest.mark.parametrize("cut", [300, 512])
@pytest.mark.parametrize("rows", [1023, 1024])
def test_relaxed_cached_and_streamed(pkg, k, arena, oracle, rows, cut):
    """One int8 token on 16-lane rows reads a launch's weights through the caches below 1 MiB and streams them past
    the caches from 1 MiB on: 1023 and 1024 rows of 1024 values, one job, then two jobs whose rows add up to the
    same (the rule counts a launch's bytes; cut at 300 the jobs' blocks are found by search, at 512 they are a grid
    row each), the corrections given and derived, every row against the oracle"""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(5 + rows)
    n, ng = 1024, 32
    frame = ((n + 4 * ng + 15) // 16) * 16
    w = rng.integers(-128, 128, rows * n).astype(np.int8)
    sums = oracle.int8_sums(w)
    ws = (rng.random(rows * ng) * 1e-3).astype(F)
    q = tile_inputs(oracle, rng, n, 1, frame, rows)
    want = oracle.matmul_q8r(q[0, :n], q[0, n:n + 4 * ng].view(F), w, ws, sums, n)
    wq, wsa, xq = arena.put(w, align=256), arena.put(ws), arena.put(q)
    for form in ("sums", "derived"):
        wca = arena.put(sums) if form == "sums" else 0
        out = arena.alloc(4 * rows, fill=np.full(rows, -7, F))
        k.matmul_q8r(out, xq, xq + n, wq, wsa, wca, n, 0, rows)
        got = arena.get(out, F, rows)
        assert same_bits(got, want), f"{rows} rows wc {form}: {first_difference(got, want)}"
        out = arena.alloc(4 * rows, fill=np.full(rows, -7, F))
        # the second job: rows cut.. of the same matrix
        table = [jobs.job("matmul_q8r", out, xq, xq + n, wq, wsa, wca, n, rows=cut),
                 jobs.job("matmul_q8r", out + 4 * cut, xq, xq + n, wq + cut * n, wsa + 4 * cut * ng,
                          wca + 4 * cut * ng if wca else 0, n, rows=rows - cut)]
        assert jobs.phase(pkg.library(), table) == 0, pkg.library().hq_last_error_message()
        got = arena.get(out, F, rows)
        assert same_bits(got, want), f"{rows} rows in two jobs wc {form}: {first_difference(got, want)}"


def test_relaxed_bytes_past_seven_bits(k, arena):
    """Activation bytes 128..255 lie outside the reference's domain (its relaxed dot is machine-dependent there):
    libhq takes every byte as a signed int8, so the token kernel and the prompt tile still agree to the bit."""
    rng = np.random.default_rng(5)
    rows, ng, count = 40, 9, 20
    n = 32 * ng
    frame = ((n + 4 * ng + 15) // 16) * 16
    w = rng.integers(-128, 128, rows * n).astype(np.int8)
    ws = (rng.random(rows * ng) * 1e-3).astype(F)
    wc = rng.integers(-200000, 200000, rows * ng).astype(np.int32)
    q = np.zeros((count, frame), np.uint8)
    q[:, :n] = rng.integers(0, 256, (count, n))
    q[:, n:n + 4 * ng] = (rng.random((count, ng)) * 1e-2).astype(F).view(np.uint8)
    wq, wsa, xq = arena.put(w), arena.put(ws), arena.put(q)
    for wca in (arena.put(wc), 0):
        tile = arena.alloc(4 * rows * count)
        k.matmul_q8r_tile(tile, xq, xq + n, wq, wsa, wca, n, 0, rows, count, 4 * rows, frame)
        got = arena.get(tile, F, rows * count).reshape(count, rows)
        for t in range(count):
            one = arena.alloc(4 * rows)
            k.matmul_q8r(one, xq + t * frame, xq + t * frame + n, wq, wsa, wca, n, 0, rows)
            want = arena.get(one, F, rows)
            assert same_bits(got[t], want), f"token {t} wc {bool(wca)}: {first_difference(got[t], want)}"


@pytest.mark.parametrize("count", [2, 4, 5, 16, 40])
@pytest.mark.parametrize("ng", [13, 16])
def test_q6r_many_tokens(pkg, arena, oracle, count, ng):
    """matmul_q6r over a prompt (no tile in the reference: a call a token, jobs.ts:471-475) through hq_phase, with
    the corrections given, moved and derived (wc = NULL); 13 groups a row (the prompt tile loads a stage's scales four
    bytes a lane) and 16 (sixteen bytes a lane)"""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(77 + count + 1000 * ng)
    rows = 90
    n = 32 * ng
    frame = ((n + 4 * ng + 15) // 16) * 16
    v = (4 * rng.integers(-32, 32, rows * n)).astype(np.int8)
    packed = pack6(v)
    ws = (rng.random(rows * ng) * 1e-3).astype(F)
    sums = oracle.six_sums(packed)
    moved = sums.copy()
    moved[[5, 600, rows * ng - 1]] += np.array([3, -64, 1 << 20], np.int32)
    q = tile_inputs(oracle, rng, n, count, frame, rows)
    wq, wsa, xq = arena.put(packed, align=256), arena.put(ws), arena.put(q)
    for form, wc in (("six_sums", sums), ("moved", moved), ("derived", None)):
        out = arena.alloc(4 * rows * count, fill=np.full(rows * count, -7, F))
        job = jobs.job("matmul_q6r", out, xq, xq + n, wq, wsa, 0 if wc is None else arena.put(wc), n, rows=rows,
                       count=count, os=4 * rows, as_=frame, bs=frame)
        assert jobs.phase(pkg.library(), [job]) == 0, pkg.library().hq_last_error_message()
        got = arena.get(out, F, rows * count).reshape(count, rows)
        for t in range(count):
            want = oracle.matmul_q6r(q[t, :n], q[t, n:n + 4 * ng].view(F), packed, ws, sums if wc is None else wc, n)
            assert same_bits(got[t], want), f"wc {form} token {t}: {first_difference(got[t], want)}"


def tile_rows(rows, token_tiles, cus):
    """the rows of the prompt kernel's tile for a launch (gemm.hip's short_tiles: 32-row tiles where their rounds of
    the 3 x CU block slots, each 0.89 of a round of 64-row tiles over 2 x CU, at least one round either way, cost
    less)"""
    t64, t32 = -(-rows // 64) * token_tiles, -(-rows // 32) * token_tiles
    return 32 if 0.89 * max(1.0, t32 / (3 * cus)) < max(1.0, t64 / (2 * cus)) else 64


@pytest.mark.parametrize("packing", ["int8", "int6"])
@pytest.mark.parametrize("ng", [13, 16])
@pytest.mark.parametrize("height", [32, 64])
def test_relaxed_prompt_many_tiles(pkg, arena, oracle, packing, ng, height):
    """A prompt over many of the matrix cores' tiles, of both heights (32 rows: a launch of few tiles, 301 rows cut at
    5 and 299; 64 rows: enough row tiles to fill the block slots, cut at 5 and 21 short of the end): tiles starting
    off a multiple of the height, a ragged last tile, 131 tokens (a ragged third token tile), the corrections given,
    moved and derived, the scales loaded four bytes a lane (13 groups: also groups past the last four) and sixteen
    (16)."""
    import torch
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(4242 + ng + (100 if packing == "int6" else 0) + height)
    count, r0 = 131, 5
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if height == 32:
        rows, r1 = 301, 299
    else:  # 64-row tiles a little fewer than the block slots: one round of them, two of 32-row tiles
        rows = 64 * ((2 * cus) // 3 - 1) + 26
        r1 = rows - 21
    # int8 goes through the drop-in tile (a launch of rows r0..r1), int6 through a phase (rows 0..r1)
    assert tile_rows(r1 - r0 if packing == "int8" else r1, 3, cus) == height
    n = 32 * ng
    frame = ((n + 4 * ng + 15) // 16) * 16
    if packing == "int8":
        wbytes = rng.integers(-128, 128, rows * n).astype(np.int8)
        sums = oracle.int8_sums(wbytes)
        product, kind = oracle.matmul_q8r, "matmul_q8r"
    else:
        wbytes = pack6((4 * rng.integers(-32, 32, rows * n)).astype(np.int8))
        sums = oracle.six_sums(wbytes)
        product, kind = oracle.matmul_q6r, "matmul_q6r"
    ws = (rng.random(rows * ng) * 1e-3).astype(F)
    ws[7::17] = F(2.0 ** -140)
    moved = sums.copy()
    moved[rng.integers(0, rows * ng, 5)] += np.array([1, -5000, 77, 1 << 21, -3], np.int32)
    q = tile_inputs(oracle, rng, n, count, frame, rows)
    wq, wsa, xq = arena.put(wbytes, align=256), arena.put(ws), arena.put(q)
    os_ = 4 * (rows + 5)
    for form, wc in (("sums", sums), ("moved", moved), ("derived", None)):
        out = arena.alloc(os_ * count, fill=np.full(os_ * count // 4, -7, F))
        wca = 0 if wc is None else arena.put(wc)
        # int8 through the drop-in tile (rows r0..r1), int6 through a phase (a job's rows start at 0)
        if packing == "int8":
            pkg.load_kernels().matmul_q8r_tile(out, xq, xq + n, wq, wsa, wca, n, r0, r1, count, os_, frame)
        else:
            job = jobs.job(kind, out, xq, xq + n, wq, wsa, wca, n, rows=r1, count=count, os=os_, as_=frame, bs=frame)
            assert jobs.phase(pkg.library(), [job]) == 0, pkg.library().hq_last_error_message()
        lo = r0 if packing == "int8" else 0
        got = arena.get(out, F, os_ * count // 4).reshape(count, -1)
        for t in range(count):
            full = product(q[t, :n], q[t, n:n + 4 * ng].view(F), wbytes, ws, sums if wc is None else wc, n)
            want = np.full(os_ // 4, F(-7), F)
            want[lo:r1] = full[lo:r1]
            assert same_bits(got[t], want), f"{packing} ng {ng} token {t} wc {form}: {first_difference(got[t], want)}"


# ---- ternary -------------------------------------------------------------------------------------------------
def ternary_case(groups, rows=ROWS, seed=231):
    rng = LCG(seed + groups)
    n = groups * 128
    codes = np.array([rng.next() & 3 for _ in range(rows * n)], np.uint8)
    codes[:128] = 2
    if groups > 1:
        codes[n + 128:n + 256] = 0
    halves = []
    for g in range(rows * groups):
        v = 2.0 ** -20 * (1 + rng.next() % 1000) if g % 11 == 7 else (0 if g % 13 == 5 else 1e-3 * (1 + rng.next() % 1000))
        halves.append(np.float16(v))
    return n, codes, np.array(halves, np.float16).view(np.uint16), rng


def ternary_acts(rng, oracle, n, pattern=None):
    if pattern is None:
        a = np.array([(rng.next() & 255) - 128 for _ in range(n)], np.int8)
    else:
        a = pattern
    xs = np.array([F(1e-2 * (1 + rng.next() % 1000)) for _ in range(n // 32)], F)
    return oracle.interleave(a, xs)


@pytest.mark.parametrize("groups", [1, 2, 3, 4, 5, 7, 9, 24, 40, 72, 136])
@pytest.mark.parametrize("name", ["matmul_t2r", "matmul_t2"])
def test_ternary_token(k, arena, oracle, groups, name):
    """Every row length class of the token kernel: rows of 8 lanes (groups a multiple of 8, not of 16), of 16, and of
    32 (8192 weights and more); activations staged in LDS."""
    n, codes, halves, rng = ternary_case(groups)
    wq = arena.put(pack_ternary(codes))
    wsa = arena.put(halves)
    for t in range(3):
        if t == 0:
            pat = np.full(n, 127, np.int8)
            pat[64:128] = -128
        else:
            pat = None
        xq_b, area = ternary_acts(rng, oracle, n, pat)
        xq, xs = arena.put(xq_b), arena.put(area)
        full = oracle.matmul_t2r(xq_b, area, pack_ternary(codes), halves, n)
        for r0, r1 in [(0, ROWS), (0, 1), (ROWS - 1, ROWS), (3, 8), (5, 5)]:
            out = arena.alloc(4 * (ROWS + 1), fill=np.full(ROWS + 1, -7, F))
            getattr(k, name)(out, xq, xs, wq, wsa, n, r0, r1, 3)
            got = arena.get(out, F, ROWS + 1)
            want = expect_range(full, r0, r1)
            assert same_bits(got, want), f"{name} groups {groups} token {t} rows {r0}..{r1}: {first_difference(got, want)}"


def test_ternary_largest_sums(k, arena, oracle):
    """tests/ternary-check.ts:184-248: rows of one code (0..3) against activations at int8's ends."""
    groups, rows = 9, ROWS
    n = groups * 128
    codes = np.zeros(rows * n, np.uint8)
    for i in range(rows):
        codes[i * n:(i + 1) * n] = i & 3
    halves = np.array([np.float16(0.5 + 0.01 * g) for g in range(rows * groups)], np.float16).view(np.uint16)
    wq, wsa = arena.put(pack_ternary(codes)), arena.put(halves)
    patterns = [lambda j: -128, lambda j: 127, lambda j: 127 if j & 1 else -128, lambda j: -128 if j & 32 else 127,
                lambda j: 0, lambda j: -127]
    for pi, pattern in enumerate(patterns):
        for t in range(5):
            a = np.array([max(-128, min(127, -pattern(j) if t % 2 else pattern(j + t))) for j in range(n)], np.int8)
            xs = np.array([F(1e-2 * (1 + ((g + t) % 7))) for g in range(n // 32)], F)
            xq_b, area = oracle.interleave(a, xs)
            want = oracle.matmul_t2r(xq_b, area, pack_ternary(codes), halves, n)
            out = arena.alloc(4 * rows)
            k.matmul_t2r(out, arena.put(xq_b), arena.put(area), wq, wsa, n, 0, rows, 3)
            got = arena.get(out, F, rows)
            assert same_bits(got, want), f"pattern {pi} token {t}: {first_difference(got, want)}"


@pytest.mark.parametrize("count,groups", [(c, g) for c in [1, 2, 3, 4, 5, 7, 8, 9, 16, 17, 64, 65, 100]
                                          for g in [1, 3, 9]] + [(4, 136), (3, 136), (2, 40)])
def test_t2r_tile(k, arena, oracle, count, groups):
    """(4, 136): four tokens of 17408 activations are more than the token kernel stages in LDS (read through the L1)"""
    n, codes, halves, rng = ternary_case(groups, rows=70, seed=500 + count)
    rows = 70
    wbytes = pack_ternary(codes)
    wq, wsa = arena.put(wbytes), arena.put(halves)
    frame = ((n + 8 * (n // 32) + 15) // 16) * 16
    buf = np.zeros((count, frame), np.uint8)
    areas = []
    for t in range(count):
        xq_b, area = ternary_acts(rng, oracle, n)
        buf[t, :n] = xq_b.view(np.uint8)
        buf[t, n:n + area.nbytes] = area.view(np.uint8)
        areas.append((xq_b, area))
    xq = arena.put(buf)
    os_ = 4 * (rows + 5)
    for r0, r1 in [(0, rows), (2, 9), (rows - 1, rows), (3, 67)]:
        out = arena.alloc(os_ * count, fill=np.full(os_ * count // 4, -7, F))
        k.matmul_t2r_tile(out, xq, xq + n, wq, wsa, n, r0, r1, count, os_, frame, 3)
        got = arena.get(out, F, os_ * count // 4).reshape(count, -1)
        for t in range(count):
            full = oracle.matmul_t2r(areas[t][0], areas[t][1], wbytes, halves, n)
            want = np.full(os_ // 4, F(-7), F)
            want[r0:r1] = full[r0:r1]
            assert same_bits(got[t], want), f"count {count} groups {groups} rows {r0}..{r1} token {t}: " \
                                            f"{first_difference(got[t], want)}"


def ternary_tile_rows(rows, token_tiles, cus):
    """the rows of the ternary prompt tile for a launch (gemm.hip's ternary_rows: 96 where its rounds of tiles over
    the CUs, one block a CU, times 96 x 1.155 cost less than the 128-row tiles' rounds times 128)"""
    r128 = -(-(-(-rows // 128) * token_tiles) // cus)
    r96 = -(-(-(-rows // 96) * token_tiles) // cus)
    return 96 if 96 * 1.155 * r96 < 128 * r128 else 128


@pytest.mark.parametrize("height", [96, 128])
@pytest.mark.parametrize("packing", ["ternary", "binary"])
def test_signs_tile_heights(pkg, k, arena, oracle, height, packing):
    """The ternary / binary prompt tile at both heights: 96 rows (a launch of few tiles: 301 rows cut at 3 and 299, 131
    tokens) and 128 (a launch of two full rounds of 128-row tiles, sized from the device's CU count: ~32 row tiles
    of 1024 tokens, cut at 5 and 21 short of the end); 3 groups of 128, rows cut inside the tiles."""
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if height == 96:
        rows, r0, r1, count = 301, 3, 299, 131
    else:
        count = 1024
        rows = 128 * ((2 * cus) // 16) + 26
        r0, r1 = 5, rows - 21
    assert ternary_tile_rows(r1 - r0, -(-count // 64), cus) == height
    groups = 3
    if packing == "ternary":
        n, codes, halves, rng = ternary_case(groups, rows=rows, seed=900 + height)
        wbytes = pack_ternary(codes)
    else:
        n, _, wbytes, halves, rng = binary_case(groups, rows=rows, seed=900 + height)
    wq, wsa = arena.put(wbytes), arena.put(halves)
    frame = ((n + 8 * (n // 32) + 15) // 16) * 16
    buf = np.zeros((count, frame), np.uint8)
    areas = []
    for t in range(count):
        xq_b, area = ternary_acts(rng, oracle, n)
        buf[t, :n] = xq_b.view(np.uint8)
        buf[t, n:n + area.nbytes] = area.view(np.uint8)
        areas.append((xq_b, area))
    xq = arena.put(buf)
    os_ = 4 * (rows + 5)
    out = arena.alloc(os_ * count, fill=np.full(os_ * count // 4, -7, F))
    if packing == "ternary":
        k.matmul_t2r_tile(out, xq, xq + n, wq, wsa, n, r0, r1, count, os_, frame, 3)
    else:
        k.matmul_b1r_tile(out, xq, xq + n, wq, wsa, n, r0, r1, count, os_, frame, 2)
    got = arena.get(out, F, os_ * count // 4).reshape(count, -1)
    product = oracle.matmul_t2r if packing == "ternary" else oracle.matmul_b1r
    for t in range(count):
        full = product(areas[t][0], areas[t][1], wbytes, halves, n)
        want = np.full(os_ // 4, F(-7), F)
        want[r0:r1] = full[r0:r1]
        assert same_bits(got[t], want), f"{packing} height {height} token {t}: {first_difference(got[t], want)}"


# ---- binary: the ternary kernels on one bit a weight ----------------------------------------------------------
def binary_case(groups, rows=ROWS, seed=634):
    """tests/ternary-check.ts:292-305: signs (row 0 all +1, row 1 all -1), written both ways, the scales of
    ternary_case"""
    n, _, halves, rng = ternary_case(groups, rows, seed)
    bits = np.array([rng.next() & 1 for _ in range(rows * n)], np.uint8)
    bits[:n], bits[n:2 * n] = 1, 0
    return n, bits, pack_binary(bits, n), halves, rng


@pytest.mark.parametrize("groups", [1, 2, 3, 4, 5, 7, 9, 24, 40, 72, 136])
@pytest.mark.parametrize("name", ["matmul_b1r", "matmul_b1"])
def test_binary_token(k, arena, oracle, groups, name):
    """Every row length class of the token kernel (rows of 8, 16 and 32 lanes), bit for bit the oracle's binary kernel
    and the ternary kernel's on the same signs"""
    n, bits, bw, halves, rng = binary_case(groups)
    wq, wsa = arena.put(bw), arena.put(halves)
    for t in range(3):
        pat = np.where(np.arange(n) & 1, 127, -128).astype(np.int8) if t == 0 else (
            np.full(n, -128, np.int8) if t == 1 else None)
        xq_b, area = ternary_acts(rng, oracle, n, pat)
        xq, xs = arena.put(xq_b), arena.put(area)
        full = oracle.matmul_b1r(xq_b, area, bw, halves, n)
        assert same_bits(full, oracle.matmul_t2r(xq_b, area, pack_ternary(2 * bits), halves, n))
        for r0, r1 in [(0, ROWS), (0, 1), (ROWS - 1, ROWS), (3, 8), (5, 5)]:
            out = arena.alloc(4 * (ROWS + 1), fill=np.full(ROWS + 1, -7, F))
            getattr(k, name)(out, xq, xs, wq, wsa, n, r0, r1, 2)
            got = arena.get(out, F, ROWS + 1)
            want = expect_range(full, r0, r1)
            assert same_bits(got, want), f"{name} groups {groups} token {t} rows {r0}..{r1}: {first_difference(got, want)}"


@pytest.mark.parametrize("rows", [2560, 3072])
@pytest.mark.parametrize("packing", ["ternary", "binary"])
def test_signs_block_waves(k, arena, oracle, rows, packing):
    """One token's launches whose blocks of 4 waves would end in a part-empty round take 5 waves (2560 rows of 32
    lanes: 256 blocks of 10 rows) or 6 (3072: 256 of 12): every row the oracle's, rows cut at both ends"""
    rng = np.random.default_rng(rows + len(packing))
    n = 8192
    q, s = oracle.quantize_x(rng.standard_normal(n).astype(F), 0)
    xq_b, area = oracle.interleave(q.view(np.int8), s)
    halves = np.repeat((np.abs(rng.standard_normal(rows)) * 0.02 + 1e-3).astype(np.float16), n // 128).view(np.uint16)
    if packing == "ternary":
        wbytes = pack_ternary(rng.integers(0, 3, rows * n).astype(np.uint8))
        full, name, last = oracle.matmul_t2r(xq_b, area, wbytes, halves, n), "matmul_t2r", 3
    else:
        wbytes = pack_binary(rng.integers(0, 2, rows * n).astype(np.uint8), n)
        full, name, last = oracle.matmul_b1r(xq_b, area, wbytes, halves, n), "matmul_b1r", 2
    wq, wsa, xq, xs = arena.put(wbytes), arena.put(halves), arena.put(xq_b), arena.put(area)
    for r0, r1 in [(0, rows), (3, rows - 5)]:
        out = arena.alloc(4 * (rows + 1), fill=np.full(rows + 1, -7, F))
        getattr(k, name)(out, xq, xs, wq, wsa, n, r0, r1, last)
        got = arena.get(out, F, rows + 1)
        want = np.full(rows + 1, F(-7), F)
        want[r0:r1] = full[r0:r1]
        assert same_bits(got, want), f"{packing} rows {r0}..{r1}: {first_difference(got, want)}"


@pytest.mark.parametrize("count,groups", [(c, g) for c in [1, 2, 3, 4, 5, 7, 8, 9, 16, 17, 64, 65, 100]
                                          for g in [1, 3, 9]] + [(4, 136), (3, 136), (2, 40), (33, 136)])
def test_b1r_tile(k, arena, oracle, count, groups):
    """every count of tokens (the token kernel up to 4 at a time, the MFMA tiles from 16), rows cut anywhere"""
    rows = 70
    n, bits, bw, halves, rng = binary_case(groups, rows=rows, seed=700 + count)
    wq, wsa = arena.put(bw), arena.put(halves)
    frame = ((n + 8 * (n // 32) + 15) // 16) * 16
    buf = np.zeros((count, frame), np.uint8)
    acts = []
    for t in range(count):
        xq_b, area = ternary_acts(rng, oracle, n)
        buf[t, :n] = xq_b.view(np.uint8)
        buf[t, n:n + area.nbytes] = area.view(np.uint8)
        acts.append((xq_b, area))
    xq = arena.put(buf)
    os_ = 4 * (rows + 5)
    for r0, r1 in [(0, rows), (2, 9), (rows - 1, rows), (3, 67)]:
        out = arena.alloc(os_ * count, fill=np.full(os_ * count // 4, -7, F))
        k.matmul_b1r_tile(out, xq, xq + n, wq, wsa, n, r0, r1, count, os_, frame, 2)
        got = arena.get(out, F, os_ * count // 4).reshape(count, -1)
        for t in range(count):
            full = oracle.matmul_b1r(acts[t][0], acts[t][1], bw, halves, n)
            want = np.full(os_ // 4, F(-7), F)
            want[r0:r1] = full[r0:r1]
            assert same_bits(got[t], want), f"count {count} groups {groups} rows {r0}..{r1} token {t}: " \
                                            f"{first_difference(got[t], want)}"


def test_binary_phase_and_matmuls(pkg, arena, oracle):
    """binary jobs (kinds 13 and 14) in hq_phase beside ternary ones, and through hq_matmuls (quantize_x at bias 0 and
    interleave, then the phase)"""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(13)
    groups, rows, tokens = 5, 45, 3
    n = 128 * groups
    bits = rng.integers(0, 2, rows * n).astype(np.uint8)
    bw, tw = pack_binary(bits, n), pack_ternary(2 * bits)
    halves = (rng.random(rows * groups) * 0.01).astype(np.float16).view(np.uint16)
    x = rng.standard_normal((tokens, n)).astype(F)
    frame = 2 * n
    sq = arena.alloc(tokens * frame)
    outs = {name: arena.alloc(4 * rows * tokens, fill=np.full(rows * tokens, -7, F))
            for name in ("matmul_b1r", "matmul_b1", "matmul_t2r")}
    wqs = {"matmul_b1r": arena.put(bw), "matmul_b1": arena.put(bw), "matmul_t2r": arena.put(tw)}
    wsa = arena.put(halves)
    table = [jobs.job(name, outs[name], sq, sq + n, wqs[name], wsa, 0, n, rows=rows, count=tokens, os=4 * rows,
                      as_=frame, bs=frame) for name in outs]
    L = pkg.library()
    assert jobs.matmuls(L, arena.put(x), 4 * n, table) == 0, L.hq_last_error_message()
    for t in range(tokens):
        q, s = oracle.quantize_x(x[t], 0)
        xi, area = oracle.interleave(q.view(np.int8), s)
        want = oracle.matmul_b1r(xi, area, bw, halves, n)
        for name in outs:
            got = arena.get(outs[name] + 4 * rows * t, F, rows)
            assert same_bits(got, want), f"{name} token {t}: {first_difference(got, want)}"


def test_binary_x(pkg, k, arena, oracle):
    """kernels/kernel/quantize.ts:232-247 on the GPU: the oracle's bytes and scales, and the refusal (the drop-in's
    return value, and the _ex form's device word)"""
    import test_oracle
    rng = np.random.default_rng(6340)
    L = pkg.library()
    for case in range(4):
        x = test_oracle.binary_x_case(rng, groups=40 + 200 * case)
        if case == 2:
            x[128 * 7 + 5] = F(-0.999999 * abs(float(x[128 * 7])))
        if case == 3:
            x[128 * 39 + 127] = np.nan
        want_out, want_xs, want_bad = oracle.binary_x(x)
        xa = arena.put(x)
        out = arena.alloc(x.size // 8, fill=np.full(x.size // 8, 0xAA, np.uint8))
        xs = arena.alloc(4 * (x.size // 128), fill=np.full(x.size // 128, -7, F))
        assert k.binary_x(out, xs, xa, x.size) == want_bad
        assert np.array_equal(arena.get(out, np.uint8, x.size // 8), want_out), case
        got_xs = arena.get(xs, F, x.size // 128)
        assert np.array_equal(np.isnan(got_xs), np.isnan(want_xs))
        assert same_bits(np.nan_to_num(got_xs), np.nan_to_num(want_xs)), case
        word = arena.alloc(4, fill=np.zeros(1, np.int32))
        assert L.hq_binary_x_ex(out, xs, xa, x.size, word, None) == 0
        assert arena.get(word, np.int32, 1)[0] == want_bad, case


def test_quantize6_x(pkg, k, arena, oracle):
    """kernels/kernel/quantize.ts:161-182 on the GPU: the oracle's 24 bytes and scale / 4 of every group (random groups
    of every magnitude, a group of zeros, ties to even, a subnormal scale, a NaN passed over and one that makes the
    scale NaN), through the drop-in name and the _ex form"""
    rng = np.random.default_rng(1611)
    L = pkg.library()
    for groups in (1, 7, 999):
        x = (rng.standard_normal((groups, 32)) * np.exp(rng.uniform(-20, 20, (groups, 1)))).astype(F)
        if groups > 7:
            x[3] = 0.0
            x[5] = np.arange(32, dtype=F) - F(15.5)
            x[5, 31] = 31.0
            x[6, 0] = 1e-38
            x[7, 1] = np.nan  # lane 1 of groupMax: passed over
            x[8, 0] = np.nan  # lane 0: the scale is NaN
        x = x.reshape(-1)
        want_out, want_xs = oracle.quantize6_x(x)
        xa = arena.put(x)
        for form in ("drop-in", "ex"):
            out = arena.alloc(groups * 24, fill=np.full(groups * 24, 0xAA, np.uint8))
            xs = arena.alloc(4 * groups, fill=np.full(groups, -7, F))
            if form == "drop-in":
                k.quantize6_x(out, xs, xa, x.size)
            else:
                assert L.hq_quantize6_x_ex(out, xs, xa, x.size, None) == 0, L.hq_last_error_message()
            assert np.array_equal(arena.get(out, np.uint8, groups * 24), want_out), (groups, form)
            got_xs = arena.get(xs, F, groups)
            assert np.array_equal(np.isnan(got_xs), np.isnan(want_xs))
            assert same_bits(np.nan_to_num(got_xs), np.nan_to_num(want_xs)), (groups, form)


def test_ternary_x(pkg, k, arena, oracle):
    """kernels/kernel/quantize.ts:197-225 on the GPU: the oracle's codes and scales (tests/ternary-check.ts:252-258's
    groups: scales of every size, zeros, -0), and its refusals (ternary-check.ts:276-283's places), through the
    drop-in's return value and the _ex form's device word"""
    import test_oracle
    rng = np.random.default_rng(2300)
    L = pkg.library()
    cases = [(None, None), (0, 0.5), (127, 1.0000001), (128 + 63, 2), (128 * 39 + 127, np.nan), (128 * 7 + 5, -0.999999),
             (128 * 9 + 33, 0.5), (128 * 9 + 38, 0.5), (128 * 9 + 43, 0.5), (128 * 9 + 46, 0.5)]
    for at, spoil in cases:
        x = test_oracle.ternary_case(rng)
        if at is not None:
            g = at >> 7
            x[g * 128:(g + 1) * 128] = np.where(np.arange(128) % 2 == 1, 3.0, -3.0)
            x[at] = F(spoil * 3)
        want_out, want_xs, want_bad = oracle.ternary_x(x)
        xa = arena.put(x)
        out = arena.alloc(x.size // 4, fill=np.full(x.size // 4, 0xAA, np.uint8))
        xs = arena.alloc(4 * (x.size // 128), fill=np.full(x.size // 128, -7, F))
        assert k.ternary_x(out, xs, xa, x.size) == want_bad, (at, spoil)
        assert np.array_equal(arena.get(out, np.uint8, x.size // 4), want_out), (at, spoil)
        got_xs = arena.get(xs, F, x.size // 128)
        assert np.array_equal(np.isnan(got_xs), np.isnan(want_xs))
        assert same_bits(np.nan_to_num(got_xs), np.nan_to_num(want_xs)), (at, spoil)
        word = arena.alloc(4, fill=np.zeros(1, np.int32))
        assert L.hq_ternary_x_ex(out, xs, xa, x.size, word, None) == 0
        assert arena.get(word, np.int32, 1)[0] == want_bad, (at, spoil)
    # a long row: 17408 values (136 groups), the 27B down projection's
    x = (rng.integers(-1, 2, 17408) * np.repeat(rng.uniform(0.01, 1, 136), 128)).astype(F)
    want_out, want_xs, want_bad = oracle.ternary_x(x)
    out, xs = arena.alloc(x.size // 4), arena.alloc(4 * 136)
    assert k.ternary_x(out, xs, arena.put(x), x.size) == want_bad == 0
    assert np.array_equal(arena.get(out, np.uint8, x.size // 4), want_out)
    assert same_bits(arena.get(xs, F, 136), want_xs)


# ---- the order-revealing inputs of test_oracle.py, on the GPU ------------------------------------------------
@pytest.mark.parametrize("ds, es, want", [
    ([1, 1, 0, 0, -1, 0, 0, 0, 0, 0, 0, 0], [24, 0, 0, 0, 24, 0, 0, 0, 0, 0, 0, 0], 1.0),
    ([1, 0, 0, 0, 1, 0, 0, 0, -1, 0, 0, 0], [24, 0, 0, 0, 0, 0, 0, 0, 24, 0, 0, 0], 0.0),
    ([1, 1, 1, -1], [24, 0, 0, 24], 0.0),
    ([1, -1, 0, 0, 1], [24, 24, 0, 0, 0], 1.0),
    ([0, 0, 0, 0, 1, 1, -1], [0, 0, 0, 0, 24, 0, 24], 0.0),
    ([1] + [0] * 15 + [1] + [0] * 15 + [-1], [24] + [0] * 31 + [24], 0.0),
    ([1, 0, 0, 0] * 8 + [-1, 0, 0, 0], [24] + [0] * 31 + [24, 0, 0, 0], 0.0),  # each +1 lost to 2^24
])
def test_q8r_order_cases(k, arena, ds, es, want):
    xq, xs, w, ws, wc, n = models.crafted_q8r(ds, es)
    for wc_addr in (arena.put(wc), 0):
        out = arena.alloc(4)
        k.matmul_q8r(out, arena.put(xq), arena.put(xs), arena.put(w), arena.put(ws), wc_addr, n, 0, 1)
        assert arena.get(out, F, 1)[0] == F(want)
        # and through the matrix cores: the same row against 20 tokens
        count, frame = 20, ((n + 4 * len(ds) + 15) // 16) * 16
        buf = np.zeros((count, frame), np.uint8)
        buf[:, :n] = xq
        buf[:, n:n + 4 * len(ds)] = xs.view(np.uint8)
        outs = arena.alloc(4 * count)
        k.matmul_q8r_tile(outs, arena.put(buf), arena.put(buf) + n, arena.put(w), arena.put(ws), wc_addr, n, 0, 1,
                          count, 4, frame)
        assert np.all(arena.get(outs, F, count) == F(want))


# ---- a phase: several jobs, mixed kinds, one call -------------------------------------------------------------
def test_phase_matches_single_calls(pkg, k, arena, oracle):
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(21)
    n = 1024
    ng = n // 32
    x = rng.standard_normal(n).astype(F)
    q64, s64 = oracle.quantize_x(x, 64)
    q0, s0 = oracle.quantize_x(x, 0)
    xq64, xs64, xq0, xs0 = arena.put(q64), arena.put(s64), arena.put(q0), arena.put(s0)
    mats, table, wants = [], [], []
    for rows in (1536, 1024, 96):
        w = rng.integers(-127, 128, rows * n).astype(np.int8)
        ws = (np.abs(rng.standard_normal(rows * ng)) * 0.02 / 127).astype(F)
        wc = oracle.int8_sums(w)
        wq, wsa, wca = arena.put(w), arena.put(ws), arena.put(wc)
        o1, o2 = arena.alloc(4 * rows), arena.alloc(4 * rows)
        table.append(jobs.job("matmul_q8r", o1, xq64, xs64, wq, wsa, wca, n, rows=rows))
        table.append(jobs.job("matmul_q8", o2, xq0, xs0, wq, wsa, 0, n, rows=rows))
        wants.append((o1, oracle.matmul_q8r(q64, s64, w, ws, wc, n)))
        wants.append((o2, oracle.matmul_q8(q0.view(np.int8), s0, w, ws, n)))
    assert jobs.phase(pkg.library(), table) == 0, pkg.library().hq_last_error_message()
    for addr, want in wants:
        assert same_bits(arena.get(addr, F, want.size), want)


# ---- a phase's jobs as pieces of equal block counts (a job a grid row), or found through block0 ---------------
@pytest.mark.parametrize("kind, tokens, n, rows", [
    ("matmul_q8r", 1, 4096, (64, 16, 16)),   # q/k/v-shaped: 16, 4, 4 blocks of 4 rows -> 6 pieces of 4 blocks
    ("matmul_q8r", 1, 4096, (56, 56)),       # gate / up: 2 pieces
    ("matmul_q8r", 1, 4096, (64, 17)),       # 16 and 5 blocks: 21 pieces, past 8 -> through block0
    ("matmul_q8r", 4, 4096, (256, 64, 64)),  # four tokens staged: 8, 2, 2 blocks of 32 rows -> 6 pieces
    ("matmul_q8r", 4, 4096, (256, 65)),      # 8 and 3 blocks -> 11 pieces -> through block0
    ("matmul_q8r", 1, 1024, (3, 40, 200)),   # 16-lane rows, 8 a block: 1, 5, 25 blocks -> through block0
    ("matmul_t2r", 1, 1024, (128, 32, 32)),  # 8-lane rows, 32 a block: 4, 1, 1 blocks -> 6 pieces
    ("matmul_t2r", 2, 1024, (100, 33)),      # 4 and 2 blocks -> 3 pieces of 2 (the last block of each partial)
])
def test_phase_job_pieces(pkg, arena, oracle, kind, tokens, n, rows):
    """Jobs of one launch whose block counts cut into at most 8 equal pieces run as a job a grid row; others find
    their job through the first blocks of each.  Either way every row of every job is the reference's number to the
    bit, for every token, and nothing past a job's rows is written."""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(sum(rows) + 7 * tokens + n)
    ternary = kind == "matmul_t2r"
    if ternary:
        pairs = [oracle.interleave(rng.integers(-128, 128, n).astype(np.int8),
                                   (rng.random(n // 32) * 0.05 + 1e-3).astype(F)) for _ in range(tokens)]
        # a token's bytes, then its area, one frame a token (the tile kinds take one stride for both)
        frame = sframe = n + 8 * (n // 32)
        buf = np.zeros(tokens * frame, np.uint8)
        for t, (b, area) in enumerate(pairs):
            buf[t * frame:t * frame + n] = b.view(np.uint8)
            buf[t * frame + n:(t + 1) * frame] = area.view(np.uint8)
        xq = arena.put(buf)
        xs = xq + n
    else:
        qs = [oracle.quantize_x(rng.standard_normal(n).astype(F), 64) for _ in range(tokens)]
        frame = sframe = 2 * n
        buf = np.zeros(tokens * frame, np.uint8)
        for t, (q, s) in enumerate(qs):
            buf[t * frame:t * frame + n] = q.view(np.uint8)
            buf[t * frame + n:t * frame + n + 4 * (n // 32)] = s.view(np.uint8)
        xq = arena.put(buf)
        xs = xq + n
    table, wants = [], []
    for r in rows:
        if ternary:
            codes = rng.integers(0, 3, r * n).astype(np.uint8)
            w = pack_ternary(codes)
            ws = np.full(r * (n // 128), 0, np.uint16)
            ws[:] = np.array(rng.random(r) * 0.02 + 1e-3, np.float16).view(np.uint16).repeat(n // 128)
            wca = 0
        else:
            w = rng.integers(-128, 128, r * n).astype(np.int8)
            ws = (np.abs(rng.standard_normal(r * (n // 32))) * 0.02 / 127).astype(F)
            wca = 0
        out = arena.alloc(4 * (r + 1) * tokens, fill=np.full((r + 1) * tokens, -7, F))
        table.append(jobs.job(kind, out, xq, xs, arena.put(w), arena.put(ws), wca, n, rows=r, count=tokens,
                              os=4 * (r + 1), as_=frame, bs=sframe))
        for t in range(tokens):
            if ternary:
                p = pairs[t]
                full = oracle.matmul_t2r(p[0], p[1], w, ws, n)
            else:
                q, s = qs[t]
                full = oracle.matmul_q8r(q, s, w, ws, oracle.int8_sums(w), n)
            want = np.append(full, F(-7))
            wants.append((out + t * 4 * (r + 1), want, f"rows {r} token {t}"))
    L = pkg.library()
    assert jobs.phase(L, table) == 0, L.hq_last_error_message()
    for addr, want, what in wants:
        got = arena.get(addr, F, want.size)
        assert same_bits(got, want), f"{kind} {rows} {what}: {first_difference(got, want)}"


@pytest.mark.parametrize("cuts", [(0, 32, 64), (0, 8, 64), (16, 48, 64), (0, 0, 40, 64)])
def test_phase_jobs_of_one_matrix(pkg, arena, oracle, cuts):
    """Jobs that are row ranges of one matrix (the same weights and outputs; a range of no rows first, too): cut
    into pieces, every range is the reference's numbers and the rows outside every range are left as they were."""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(len(cuts) + sum(cuts))
    n, rows = 4096, 64
    q, s = oracle.quantize_x(rng.standard_normal(n).astype(F), 64)
    buf = np.concatenate([q.view(np.uint8), s.view(np.uint8)])
    xq = arena.put(buf)
    w = rng.integers(-128, 128, rows * n).astype(np.int8)
    ws = (np.abs(rng.standard_normal(rows * (n // 32))) * 0.02 / 127).astype(F)
    wq, wsa = arena.put(w), arena.put(ws)
    out = arena.alloc(4 * (rows + 1), fill=np.full(rows + 1, -7, F))
    table = [jobs.job("matmul_q8r", out + 4 * a, xq, xq + n, wq + a * n, wsa + 4 * a * (n // 32), 0, n, rows=b - a)
             for a, b in zip(cuts, cuts[1:])]
    L = pkg.library()
    assert jobs.phase(L, table) == 0, L.hq_last_error_message()
    full = oracle.matmul_q8r(q, s, w, ws, oracle.int8_sums(w), n)
    want = np.full(rows + 1, F(-7), F)
    want[cuts[0]:cuts[-1]] = full[cuts[0]:cuts[-1]]
    got = arena.get(out, F, rows + 1)
    assert same_bits(got, want), f"cuts {cuts}: {first_difference(got, want)}"


# ---- hq_matmuls: ready() into the jobs' a / b, then the phase ------------------------------------------------
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 7])
@pytest.mark.parametrize("n", [288, 4096, 17408])
def test_matmuls_relaxed(pkg, arena, oracle, tokens, n):
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(n + tokens)
    ng = n // 32
    x = rng.standard_normal((tokens, n)).astype(F)
    x[0, 32:64] = 0
    ax = arena.put(x)
    table, wants = [], []
    for kind, rows in (("matmul_q8r", 70), ("matmul_q8r_derived", 33), ("matmul_q6r", 50)):
        six = kind == "matmul_q6r"
        if six:
            v = (4 * rng.integers(-32, 32, rows * n)).astype(np.int8)
            wbytes, wc = pack6(v), oracle.six_sums(pack6(v))
        else:
            wbytes = rng.integers(-128, 128, rows * n).astype(np.int8)
            wc = oracle.int8_sums(wbytes)
        ws = (np.abs(rng.standard_normal(rows * ng)) * 0.02 / 127).astype(F)
        os_ = 4 * rows
        out = arena.alloc(os_ * tokens, fill=np.full(rows * tokens, -7, F))
        scratch = arena.alloc(tokens * 2 * n)  # where ready() puts xq / xs
        wca = 0 if kind == "matmul_q8r_derived" else arena.put(wc)
        name = "matmul_q6r" if six else "matmul_q8r"
        table.append(jobs.job(name, out, scratch, scratch + n, arena.put(wbytes), arena.put(ws), wca, n, rows=rows,
                              count=tokens, os=os_, as_=2 * n, bs=2 * n))
        for t in range(tokens):
            q, s = oracle.quantize_x(x[t], 64)
            full = (oracle.matmul_q6r if six else oracle.matmul_q8r)(q, s, wbytes, ws, wc, n)
            wants.append((out + t * os_, full, f"{kind} token {t}"))
            wants.append((scratch + t * 2 * n, q.view(np.int8), f"{kind} xq of token {t}"))
            wants.append((scratch + t * 2 * n + n, s, f"{kind} xs of token {t}"))
    # a job of no rows whose a / b are 0 (of another n, too): passed over, nothing readied into it
    table.insert(1, jobs.job("matmul_q8r", 0, 0, 0, 0, 0, 0, 2 * n, rows=0, count=tokens))
    L = pkg.library()
    assert jobs.matmuls(L, ax, 4 * n, table) == 0, L.hq_last_error_message()
    for addr, want, what in wants:
        got = arena.get(addr, want.dtype, want.size)
        assert same_bits(got, want), f"{what}: {first_difference(got, want)}"


@pytest.mark.parametrize("tokens", [1, 3])
def test_matmuls_relaxed_many_tiles(pkg, arena, oracle, tokens):
    """jobs of tens of thousands of rows (thousands of 8-row tiles) sharing one pair of a / b, across the boundary
    of two jobs of a launch, with the groups past the fours (n = 320: 10 groups)"""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(900 + tokens)
    n = 320
    ng = n // 32
    x = rng.standard_normal((tokens, n)).astype(F)
    ax = arena.put(x)
    scratch = arena.alloc(tokens * 2 * n)  # every job's a / b
    table, wants = [], []
    for name, rows, derived in (("matmul_q8r", 30011, False), ("matmul_q8r", 9000, False),
                                ("matmul_q8r", 25003, True), ("matmul_q6r", 14000, False)):
        six = name == "matmul_q6r"
        if six:
            v = (4 * rng.integers(-32, 32, rows * n)).astype(np.int8)
            wbytes, wc = pack6(v), oracle.six_sums(pack6(v))
        else:
            wbytes = rng.integers(-128, 128, rows * n).astype(np.int8)
            wc = oracle.int8_sums(wbytes)
        ws = (np.abs(rng.standard_normal(rows * ng)) * 0.02 / 127).astype(F)
        os_ = 4 * rows
        out = arena.alloc(os_ * tokens, fill=np.full(rows * tokens, -7, F))
        table.append(jobs.job(name, out, scratch, scratch + n, arena.put(wbytes), arena.put(ws),
                              0 if derived else arena.put(wc), n, rows=rows, count=tokens, os=os_, as_=2 * n,
                              bs=2 * n))
        for t in range(tokens):
            q, sc = oracle.quantize_x(x[t], 64)
            full = (oracle.matmul_q6r if six else oracle.matmul_q8r)(q, sc, wbytes, ws, wc, n)
            wants.append((out + t * os_, full, f"{name} {rows} rows token {t}"))
    L = pkg.library()
    assert jobs.matmuls(L, ax, 4 * n, table) == 0, L.hq_last_error_message()
    for addr, want, what in wants:
        got = arena.get(addr, F, want.size)
        assert same_bits(got, want), f"{what}: {first_difference(got, want)}"


@pytest.mark.parametrize("tokens", [1, 2, 4, 6])
@pytest.mark.parametrize("n", [288, 4096, 14336])
def test_matmuls_is_quantize_then_phase(pkg, arena, oracle, tokens, n):
    """hq_matmuls of the relaxed kinds (matmulsAlike: the input readied into the jobs' a / b, then the phase): its
    outputs and readied a / b against quantize_x then hq_phase on the same inputs, to the bit, over groups whose scale
    is NaN (lane 0 of groupMax), whose NaN is passed over (lane 1), of infinities, zeros, -0 and subnormals; jobs with
    and without wc, int8 and int6, two jobs sharing one a / b (readied once), one of 1000 rows; every row against the
    oracle too (NaN where it has NaN)"""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(7 * n + tokens)
    ng = n // 32
    x = (rng.standard_normal((tokens, n)) * np.exp(rng.uniform(-8, 8, (tokens, ng, 1))).repeat(32, 1).reshape(
        tokens, n)).astype(F)
    x[0, 0:32] = 0.0
    x[0, 33] = -0.0
    x[0, 64 + 1] = np.nan        # passed over: the group's scale from the other lanes
    x[0, 96 + 7] = np.inf
    x[-1, 128:160] = 1e-40       # a subnormal group
    x[-1, 160] = np.nan          # lane 0 of groupMax: the scale is NaN
    ax = arena.put(x)
    L = pkg.library()
    frame = 2 * n
    shared = arena.alloc(tokens * frame)
    specs = []   # (name, rows, wc?, a / b)
    for name, rows, with_wc, ab in (("matmul_q8r", 70, True, None), ("matmul_q8r", 33, False, None),
                                    ("matmul_q8r", 1000, True, shared), ("matmul_q8r", 9, True, shared),
                                    ("matmul_q6r", 50, True, None), ("matmul_q6r", 17, False, None)):
        six = name == "matmul_q6r"
        if six:
            v = (4 * rng.integers(-32, 32, rows * n)).astype(np.int8)
            wbytes, wc = pack6(v), oracle.six_sums(pack6(v))
        else:
            wbytes = rng.integers(-128, 128, rows * n).astype(np.int8)
            wc = oracle.int8_sums(wbytes)
        ws = (np.abs(rng.standard_normal(rows * ng)) * 0.02 / 127).astype(F)
        specs.append((name, rows, six, wbytes, wc, arena.put(wbytes), arena.put(ws), arena.put(wc) if with_wc else 0,
                      ws, ab))
    runs = {}
    for form in ("matmuls", "two launches"):
        table, outs, abs_ = [], [], []
        for name, rows, six, wbytes, wc, wa, wsa, wca, ws, ab in specs:
            out = arena.alloc(4 * rows * tokens, fill=np.full(rows * tokens, -7, F))
            if ab is None or form == "two launches":
                ab = arena.alloc(tokens * frame, fill=np.full(tokens * frame, 0xAA, np.uint8))
            table.append(jobs.job(name, out, ab, ab + n, wa, wsa, wca, n, rows=rows, count=tokens, os=4 * rows,
                                  as_=frame, bs=frame))
            outs.append(out)
            abs_.append(ab)
        if form == "matmuls":
            assert jobs.matmuls(L, ax, 4 * n, table) == 0, L.hq_last_error_message()
        else:
            for ab in abs_:
                assert L.hq_quantize_x_batch(ab, ab + n, ax, n, 64, tokens, frame, 4 * n, None) == 0
            assert jobs.phase(L, table) == 0, L.hq_last_error_message()
        runs[form] = ([arena.get(o, F, r * tokens) for o, (_, r, *_) in zip(outs, specs)],
                      [(arena.get(ab, np.uint8, tokens * frame).reshape(tokens, frame)) for ab in abs_])
    for i, (name, rows, six, wbytes, wc, wa, wsa, wca, ws, _) in enumerate(specs):
        got, want = runs["matmuls"][0][i], runs["two launches"][0][i]
        assert np.array_equal(np.isnan(got), np.isnan(want)), name
        assert same_bits(np.nan_to_num(got), np.nan_to_num(want)), f"{name} {rows}: {first_difference(got, want)}"
        ga, wa_ = runs["matmuls"][1][i], runs["two launches"][1][i]
        assert np.array_equal(ga[:, :n], wa_[:, :n]), f"{name} {rows}: readied bytes"
        gs, ws_ = ga[:, n:n + 4 * ng].copy().view(F), wa_[:, n:n + 4 * ng].copy().view(F)
        assert np.array_equal(np.isnan(gs), np.isnan(ws_)) and same_bits(np.nan_to_num(gs), np.nan_to_num(ws_))
        for t in range(tokens):
            q, sc = oracle.quantize_x(x[t], 64)
            full = (oracle.matmul_q6r if six else oracle.matmul_q8r)(q, sc, wbytes, ws, wc, n)
            g = got[t * rows:(t + 1) * rows]
            assert np.array_equal(np.isnan(g), np.isnan(full)), f"{name} {rows} token {t}"
            assert same_bits(np.nan_to_num(g), np.nan_to_num(full)), f"{name} {rows} token {t}: " \
                f"{first_difference(g, full)}"


@pytest.mark.parametrize("tokens", [1, 3, 5])
def test_matmuls_plain_and_ternary(pkg, arena, oracle, tokens):
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(40 + tokens)
    n, rows = 1024, 40
    ng = n // 32
    x = rng.standard_normal((tokens, n)).astype(F)
    ax = arena.put(x)
    w = rng.integers(-127, 128, rows * n).astype(np.int8)
    ws = (np.abs(rng.standard_normal(rows * ng)) * 0.02 / 127).astype(F)
    codes = rng.integers(0, 3, rows * n).astype(np.uint8)
    halves = (np.abs(rng.standard_normal(rows * (n // 128))) * 0.01).astype(np.float16).view(np.uint16)
    frame = 2 * n
    sq, st = arena.alloc(tokens * frame), arena.alloc(tokens * frame)
    oq, ot = arena.alloc(4 * rows * tokens), arena.alloc(4 * rows * tokens)
    table = [jobs.job("matmul_q8", oq, sq, sq + n, arena.put(w), arena.put(ws), 0, n, rows=rows, count=tokens,
                      os=4 * rows, as_=frame, bs=frame),
             jobs.job("matmul_t2r", ot, st, st + n, arena.put(pack_ternary(codes)), arena.put(halves), 0, n, rows=rows,
                      count=tokens, os=4 * rows, as_=frame, bs=frame)]
    L = pkg.library()
    assert jobs.matmuls(L, ax, 4 * n, table) == 0, L.hq_last_error_message()
    for t in range(tokens):
        q0, s0 = oracle.quantize_x(x[t], 0)
        want = oracle.matmul_q8(q0.view(np.int8), s0, w, ws, n)
        assert same_bits(arena.get(oq + 4 * rows * t, F, rows), want)
        xi, area = oracle.interleave(q0.view(np.int8), s0)
        want_t = oracle.matmul_t2r(xi, area, pack_ternary(codes), halves, n)
        assert same_bits(arena.get(ot + 4 * rows * t, F, rows), want_t)


# ---- the ceilings -------------------------------------------------------------------------------------------------
def test_ceiling_read_reads_every_byte(pkg, arena):
    """hq_ceiling_read stores a lane's fold only when it equals 0x9e3779b9: a buffer whose only nonzero word is that
    value, in the partial last block (16 KB + 48 bytes: three 16-byte pieces past the first block), makes lane 0 of
    that block store it; an all-zero buffer stores nothing"""
    L = pkg.library()
    size = 16384 + 48
    for where in (None, 16384, 16384 + 32):
        words = np.zeros(size // 4, np.uint32)
        if where is not None:
            words[where // 4] = 0x9E3779B9
        buf = arena.put(words)
        sink = arena.alloc(1024, fill=np.zeros(256, np.uint32))
        assert L.hq_ceiling_read(buf, size, sink, None) == 0, L.hq_last_error_message()
        got = arena.get(sink, np.uint32, 256)
        want = np.zeros(256, np.uint32)
        if where is not None:  # uint4 1024 + 2 q is lane 2 q of the last block's first wave
            want[(where - 16384) // 16] = 0x9E3779B9
        assert np.array_equal(got, want), (where, np.nonzero(got))


def test_ceiling_mfma_runs(pkg, arena):
    L = pkg.library()
    sink = arena.alloc(1024, fill=np.zeros(256, np.int32))
    assert L.hq_ceiling_mfma(4, 3, sink, None) == 0, L.hq_last_error_message()
    assert not arena.get(sink, np.int32, 256).any()


@pytest.mark.parametrize("form", [0, 1])
def test_ceiling_epilogue_runs(pkg, arena, form):
    """both prompt-tile epilogues on registers (an odd number of groups, blocks of 4 waves) run and store nothing"""
    L = pkg.library()
    sink = arena.alloc(1024, fill=np.zeros(256, np.int32))
    assert L.hq_ceiling_epilogue(form, 8, 7, sink, None) == 0, L.hq_last_error_message()
    assert not arena.get(sink, np.int32, 256).any()
