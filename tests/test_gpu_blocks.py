"""llama.cpp's blocks of 256 weights on the GPU (kernels/blocks/): every kernel through the C-ABI, bit for bit against
the oracle (oracle/oracle.c, pinned in test_oracle.py against a model of the converter's readers, and in
test_blocks_digests.py to the reference's own digests of what its readers read), for all ten types, with random
codebooks and random blocks of sane scales (tests/blocks_model.py), and the reader on the digests' blocks with
llama.cpp's codebooks."""
import numpy as np
import pytest

import blocks_model as bm
from gpu_util import Arena, first_difference, same_bits
from models import F

pytestmark = pytest.mark.gpu
TYPES = sorted(bm.TYPES.items(), key=lambda kv: kv[1])


@pytest.fixture(scope="module")
def k(pkg):
    import torch
    assert torch.cuda.is_available(), "the GPU tests need a GPU"
    return pkg.load_kernels()


@pytest.fixture(scope="module")
def arena():
    return Arena(1 << 28)


@pytest.fixture(autouse=True)
def fresh(arena):
    arena.reset()
    yield


@pytest.fixture(scope="module")
def setup(oracle):
    rng = np.random.default_rng(3630)
    row = bm.codebooks(rng)
    return row, oracle.sb_tables(row)


def put_tables(k, arena, row):
    """the tables made on the GPU from the codebooks row (sb_tables), and its return value"""
    area = arena.alloc(34992 + 64, fill=np.full(34992 + 64, 0xAA, np.uint8))
    assert k.sb_tables(area, arena.put(row)) == 34992
    return area


def token_area(oracle, rng, n, scale=1.0):
    x = (rng.standard_normal(n) * scale).astype(F)
    q, s = oracle.quantize_x(x, 0)
    q = q.view(np.int8)
    return q, oracle.sums_x(q, s)


def test_sb_tables_and_sums_x(pkg, k, arena, oracle, setup):
    row, tab = setup
    area = put_tables(k, arena, row)
    got = arena.get(area, np.uint8, 34992 + 64)
    assert np.array_equal(got[:34992], tab) and np.all(got[34992:] == 0xAA)
    rng = np.random.default_rng(1)
    for n in (256, 4096, 17408):
        count, frame = 3, ((2 * n + 15) // 16) * 16
        buf = np.zeros(count * frame, np.uint8)
        wants = []
        for t in range(count):
            q, area_t = token_area(oracle, rng, n)
            buf[t * frame:t * frame + n] = q.view(np.uint8)
            buf[t * frame + n:t * frame + n + 4 * (n // 32)] = area_t[:4 * (n // 32)]
            wants.append(area_t)
        b = arena.put(buf)
        assert pkg.library().hq_sums_x_batch(b + n, b, n, count, frame, None) == 0
        for t in range(count):
            got = arena.get(b + t * frame + n, np.uint8, wants[t].size)
            assert np.array_equal(got, wants[t]), (n, t)


@pytest.mark.parametrize("name,t", TYPES)
def test_sb_row(k, arena, oracle, setup, name, t):
    row, tab = setup
    area = put_tables(k, arena, row)
    rng = np.random.default_rng(t)
    for tiny in (False, True):
        blocks = bm.random_blocks(rng, t, 9, tiny)
        n = 256 * len(blocks)
        w = arena.alloc(blocks.size + 2) + 2  # 2 bytes into a word
        arena.write(w, blocks)
        out = arena.alloc(4 * n)
        k.sb_row(out, w, area, n, t)
        got = arena.get(out, F, n)
        want = oracle.sb_row(blocks.reshape(-1), tab, n, t)
        assert same_bits(got, want), f"{name} tiny {tiny}: {first_difference(got, want)}"


@pytest.mark.parametrize("name,t", TYPES)
def test_sb_row_on_the_references_digest_blocks(k, arena, oracle, name, t):
    """the reference's golden vectors (tests/fixtures/superblocks.json "read"; test_blocks_digests.py): the GPU's
    reader on the digests' 2000 SHAKE-256 blocks with llama.cpp's codebooks (tables made on the device) is the
    oracle's to the bit, and gives the reference's digest wherever the kernels' and the converter's widening of the
    float16 scales agree (every block whose scales are finite)"""
    from test_blocks_digests import BLOCKS, DIGESTS, codebooks, digest, model_floats, shake_blocks
    row = codebooks()
    area = put_tables(k, arena, row)
    blocks = shake_blocks(name)
    n = 256 * BLOCKS
    w = arena.alloc(blocks.size + 2) + 2  # 2 bytes into a word
    arena.write(w, blocks)
    out = arena.alloc(4 * n)
    k.sb_row(out, w, area, n, t)
    got = arena.get(out, F, n)
    want = oracle.sb_row(blocks.reshape(-1), oracle.sb_tables(row), n, t)
    assert same_bits(got, want), f"{name}: {first_difference(got, want)}"
    ieee, kernel = model_floats(name, row, bm.ieee_half), model_floats(name, row, bm.kernel_half)
    same = (np.nan_to_num(ieee, nan=0.0).view(np.uint32) == kernel.view(np.uint32)).reshape(BLOCKS, 256).all(1)
    assert digest(np.where(np.repeat(same, 256), got, ieee)) == DIGESTS[name]


@pytest.mark.parametrize("name,t", TYPES)
@pytest.mark.parametrize("nb", [1, 3, 20, 68])
def test_matmul_sbr(k, arena, oracle, setup, name, t, nb):
    """a token, rows cut anywhere, both alignments of the weights, and the plain kernel's same numbers"""
    row, tab = setup
    area = put_tables(k, arena, row)
    rng = np.random.default_rng(1000 * t + nb)
    rows, n = 37, 256 * nb
    blocks = bm.random_blocks(rng, t, rows * nb)
    wbytes = blocks.reshape(-1)
    for shift in (0, 2):
        w = arena.alloc(wbytes.size + 4) + shift
        arena.write(w, wbytes)
        for trial in range(2):
            q, act = token_area(oracle, rng, n, 1 + 5 * trial)
            xq, xs = arena.put(q), arena.put(act)
            full = oracle.matmul_sbr(q, act, wbytes, tab, n, t)
            for name_k in ("matmul_sbr", "matmul_sb"):
                for r0, r1 in [(0, rows), (0, 1), (rows - 1, rows), (3, 20), (5, 5)]:
                    out = arena.alloc(4 * (rows + 1), fill=np.full(rows + 1, -7, F))
                    getattr(k, name_k)(out, xq, xs, w, area, n, r0, r1, t)
                    got = arena.get(out, F, rows + 1)
                    want = np.full(rows + 1, F(-7), F)
                    want[r0:r1] = full[r0:r1]
                    assert same_bits(got, want), \
                        f"{name_k} {name} nb {nb} shift {shift} trial {trial} rows {r0}..{r1}: {first_difference(got, want)}"


@pytest.mark.parametrize("name,t", TYPES)
def test_matmul_sbr_tile(k, arena, oracle, setup, name, t):
    """1..100 tokens (4 a launch below 16, the matrix-core tile from 16: one, two and partial tiles of 64),
    rows cut anywhere; matmul_sbw_tile the same numbers"""
    row, tab = setup
    area = put_tables(k, arena, row)
    rng = np.random.default_rng(77 + t)
    rows, nb = 45, 5
    n = 256 * nb
    blocks = bm.random_blocks(rng, t, rows * nb)
    wbytes = blocks.reshape(-1)
    w = arena.put(wbytes)
    frame = ((n + n // 2 + 15) // 16) * 16
    tokens = 100
    buf = np.zeros(tokens * frame, np.uint8)
    fulls = []
    for tk in range(tokens):
        q, act = token_area(oracle, rng, n)
        buf[tk * frame:tk * frame + n] = q.view(np.uint8)
        buf[tk * frame + n:tk * frame + n + act.size] = act
        fulls.append(oracle.matmul_sbr(q, act, wbytes, tab, n, t))
    xq = arena.put(buf)
    os_ = 4 * (rows + 3)
    for count in (1, 2, 3, 4, 5, 8, 9, 16, 17, 64, 65, 100):
        for r0, r1 in [(0, rows), (2, 9), (rows - 1, rows)]:
            for form in ("matmul_sbr_tile", "matmul_sbw_tile"):
                out = arena.alloc(os_ * count, fill=np.full(os_ * count // 4, -7, F))
                args = (out, xq, xq + n, w, area, n, r0, r1, count, os_, frame, t)
                if form == "matmul_sbw_tile":
                    args = args + (0,)
                getattr(k, form)(*args)
                got = arena.get(out, F, os_ * count // 4).reshape(count, -1)
                for tk in range(count):
                    want = np.full(os_ // 4, F(-7), F)
                    want[r0:r1] = fulls[tk][r0:r1]
                    assert same_bits(got[tk], want), \
                        f"{form} {name} count {count} rows {r0}..{r1} token {tk}: {first_difference(got[tk], want)}"


@pytest.mark.parametrize("name,t", TYPES)
def test_matmul_sbr_tile_rows(k, arena, oracle, setup, name, t):
    """the matrix-core tile over several tiles of rows and two of tokens, row ranges that start and end inside a
    tile, the weights 2 bytes into a word"""
    row, tab = setup
    area = put_tables(k, arena, row)
    rng = np.random.default_rng(500 + t)
    rows, nb, tokens = 150, 3, 80
    n = 256 * nb
    wbytes = bm.random_blocks(rng, t, rows * nb).reshape(-1)
    w = arena.put(np.concatenate([np.zeros(2, np.uint8), wbytes])) + 2
    frame = ((n + n // 2 + 15) // 16) * 16
    buf = np.zeros(tokens * frame, np.uint8)
    fulls = []
    for tk in range(tokens):
        q, act = token_area(oracle, rng, n, scale=1.0 + tk % 7)
        buf[tk * frame:tk * frame + n] = q.view(np.uint8)
        buf[tk * frame + n:tk * frame + n + act.size] = act
        fulls.append(oracle.matmul_sbr(q, act, wbytes, tab, n, t))
    xq = arena.put(buf)
    os_ = 4 * (rows + 1)
    for r0, r1 in [(0, rows), (5, rows), (64, 129)]:
        out = arena.alloc(os_ * tokens, fill=np.full(os_ * tokens // 4, -7, F))
        k.matmul_sbr_tile(out, xq, xq + n, w, area, n, r0, r1, tokens, os_, frame, t)
        got = arena.get(out, F, os_ * tokens // 4).reshape(tokens, -1)
        for tk in range(tokens):
            want = np.full(os_ // 4, F(-7), F)
            want[r0:r1] = fulls[tk][r0:r1]
            assert same_bits(got[tk], want), f"{name} rows {r0}..{r1} token {tk}: {first_difference(got[tk], want)}"


@pytest.mark.parametrize("name,t", TYPES)
def test_matmul_sbr_tile_wide(k, arena, oracle, setup, name, t):
    """enough rows that the launch takes the wide tiles (a block of 128 tokens for one-scale-a-group types without
    sums, 64 for the others: at least two blocks a compute unit), 130 tokens (a partial second tile): every token of
    the first and last 64 rows, and every row of seven tokens"""
    row, tab = setup
    area = put_tables(k, arena, row)
    rng = np.random.default_rng(900 + t)
    rows, n, tokens = 16400, 256, 130
    wbytes = bm.random_blocks(rng, t, rows).reshape(-1)
    w = arena.put(wbytes)
    frame = ((n + n // 2 + 15) // 16) * 16
    buf = np.zeros(tokens * frame, np.uint8)
    acts = []
    for tk in range(tokens):
        q, act = token_area(oracle, rng, n, scale=1.0 + tk % 5)
        buf[tk * frame:tk * frame + n] = q.view(np.uint8)
        buf[tk * frame + n:tk * frame + n + act.size] = act
        acts.append((q, act))
    xq = arena.put(buf)
    os_ = 4 * rows
    out = arena.alloc(os_ * tokens, fill=np.full(rows * tokens, -7, F))
    k.matmul_sbr_tile(out, xq, xq + n, w, area, n, 0, rows, tokens, os_, frame, t)
    got = arena.get(out, F, rows * tokens).reshape(tokens, rows)
    for tk, (q, act) in enumerate(acts):
        for r0, r1 in ((0, 64), (rows - 64, rows)):
            want = oracle.matmul_sbr(q, act, wbytes, tab, n, t, r0, r1)[r0:r1]
            assert same_bits(got[tk, r0:r1], want), f"{name} token {tk} rows {r0}..{r1}: {first_difference(got[tk, r0:r1], want)}"
    for tk in (0, 31, 64, 100, 127, 128, 129):
        want = oracle.matmul_sbr(*acts[tk], wbytes, tab, n, t)
        assert same_bits(got[tk], want), f"{name} token {tk}: {first_difference(got[tk], want)}"


def test_phase_and_matmuls_of_blocks(pkg, k, arena, oracle, setup):
    """jobs of kinds 10, 11, 12 of several types in one hq_phase, and hq_matmuls (quantize_x at bias 0 and sums_x,
    then the phase) for three tokens"""
    from pyodide_llm_amd import jobs
    row, tab = setup
    area = put_tables(k, arena, row)
    rng = np.random.default_rng(12)
    n, tokens = 768, 3
    frame = ((n + n // 2 + 15) // 16) * 16
    x = rng.standard_normal((tokens, n)).astype(F)
    sq = arena.alloc(tokens * frame)
    table, wants = [], []
    for kind, (name, t, rows) in zip(("matmul_sbr", "matmul_sb", "matmul_sbw", "matmul_sbr"),
                                     (("Q4_K", 12, 33), ("IQ2_XXS", 16, 20), ("IQ1_M", 29, 17), ("IQ4_XS", 23, 50))):
        blocks = bm.random_blocks(rng, t, rows * (n // 256))
        out = arena.alloc(4 * rows * tokens, fill=np.full(rows * tokens, -7, F))
        table.append(jobs.job(kind, out, sq, sq + n, arena.put(blocks), area, t, n, rows=rows, count=tokens,
                              os=4 * rows, as_=frame, bs=frame))
        for tk in range(tokens):
            q, s = oracle.quantize_x(x[tk], 0)
            act = oracle.sums_x(q.view(np.int8), s)
            wants.append((out + 4 * rows * tk, oracle.matmul_sbr(q.view(np.int8), act, blocks.reshape(-1), tab, n, t),
                          f"{kind} {name} token {tk}"))
    L = pkg.library()
    assert jobs.matmuls(L, arena.put(x), 4 * n, table) == 0, L.hq_last_error_message()
    for addr, want, what in wants:
        got = arena.get(addr, F, want.size)
        assert same_bits(got, want), f"{what}: {first_difference(got, want)}"
    # and hq_phase on the activations hq_matmuls left
    for addr, want, _ in wants:
        arena.write(addr, np.full(want.size, -7, F))
    assert jobs.phase(L, table) == 0, L.hq_last_error_message()
    for addr, want, what in wants:
        assert same_bits(arena.get(addr, F, want.size), want), what


@pytest.mark.parametrize("name,t", [("Q4_K", 12), ("IQ4_XS", 23)])
@pytest.mark.parametrize("nb", [16, 56])
def test_matmul_sbr_coalesced_batches(pkg, k, arena, oracle, setup, name, t, nb):
    """the types whose token steps are read as coalesced 16-byte loads and handed to the lanes through LDS (blocks of
    144 and 136 bytes, one token staged, every row of the launch starting on 16 bytes): three jobs of one token in
    one hq_phase (rows not a multiple of a wave's), 16- and 64-lane rows; then the same with one matrix 2 bytes into
    a word, which takes the whole launch back to a lane's own loads"""
    from pyodide_llm_amd import jobs
    row, tab = setup
    area = put_tables(k, arena, row)
    rng = np.random.default_rng(4400 + t + nb)
    n = 256 * nb
    q, act = token_area(oracle, rng, n)
    xq, xs = arena.put(q), arena.put(act)
    L = pkg.library()
    for shifts in ((0, 0, 0), (0, 2, 0)):
        table, wants = [], []
        for rows, shift in zip((37, 50, 9), shifts):
            wbytes = bm.random_blocks(rng, t, rows * nb).reshape(-1)
            w = arena.alloc(wbytes.size + 16) + shift
            arena.write(w, wbytes)
            out = arena.alloc(4 * (rows + 1), fill=np.full(rows + 1, -7, F))
            table.append(jobs.job("matmul_sbr", out, xq, xs, w, area, t, n, rows=rows))
            want = np.full(rows + 1, F(-7), F)
            want[:rows] = oracle.matmul_sbr(q, act, wbytes, tab, n, t)
            wants.append((out, want, f"{name} nb {nb} shifts {shifts} rows {rows}"))
        assert jobs.phase(L, table) == 0, L.hq_last_error_message()
        for out, want, what in wants:
            got = arena.get(out, F, want.size)
            assert same_bits(got, want), f"{what}: {first_difference(got, want)}"


def test_signed_dots(k, arena):
    rng = np.random.default_rng(9)
    a = rng.integers(-128, 128, 16).astype(np.int8)
    b = rng.integers(-128, 128, 16).astype(np.int8)
    a[0], b[0] = -128, -128
    out = arena.alloc(16)
    k.signed_dots(out, arena.put(a), arena.put(b))
    want = (a.astype(np.int32) * b.astype(np.int32)).reshape(4, 4).sum(1)
    assert np.array_equal(arena.get(out, np.int32, 4), want)
