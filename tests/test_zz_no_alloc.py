"""hq_matmuls_static (the form of hq_matmuls that allocates nothing: the readied activations in the library's own
static staging, not the jobs' a / b) against hq_matmuls on the same inputs, through the C-ABI, to the bit: two calls
in a row, the second with a smaller input, every kind of job the staging serves (relaxed int8 with and without the
caller's corrections, relaxed int6, plain int8, ternary, binary, llama.cpp's blocks, whose sums_x fills the staging
frame's scale area), a prompt through the matrix-core tiles and a decode through the token kernels; and the refusal
of inputs past the staging's 4 MiB."""
import numpy as np
import pytest

import blocks_model as bm
from gpu_util import Arena, first_difference, same_bits
from streams import pack6, pack_binary, pack_ternary

pytestmark = pytest.mark.gpu
F = np.float32
STAGING = 4 << 20


@pytest.fixture(scope="module")
def arena():
    import torch
    assert torch.cuda.is_available(), "the GPU tests need a GPU"
    return Arena(1 << 27)


def staged_frame(n):
    return -(-n // 256) * 256 + -(-(n // 2) // 256) * 256


def phase_of(pkg, arena, oracle, rng, n, tokens, rows):
    """jobs of eight kinds over one input: (x on the device, [(job's numbers without outputs)], output sizes)"""
    ng = n // 32
    specs = []
    w8 = rng.integers(-128, 128, rows * n).astype(np.int8)
    ws = (np.abs(rng.standard_normal(rows * ng)) * 0.02 / 127).astype(F)
    aw8, aws = arena.put(w8), arena.put(ws)
    specs.append(("matmul_q8r", aw8, aws, arena.put(oracle.int8_sums(w8))))
    specs.append(("matmul_q8r", aw8, aws, 0))  # corrections derived in the kernel
    v6 = (4 * rng.integers(-32, 32, rows * n)).astype(np.int8)
    p6 = pack6(v6)
    specs.append(("matmul_q6r", arena.put(p6), aws, arena.put(oracle.six_sums(p6))))
    specs.append(("matmul_q8", aw8, aws, 0))
    codes = rng.integers(0, 3, rows * n).astype(np.uint8)
    halves = (np.abs(rng.standard_normal(rows * (n // 128))) * 0.01).astype(np.float16).view(np.uint16)
    specs.append(("matmul_t2r", arena.put(pack_ternary(codes)), arena.put(halves), 0))
    signs = rng.integers(0, 2, rows * n).astype(np.uint8)
    specs.append(("matmul_b1r", arena.put(pack_binary(signs, n)), arena.put(halves), 0))
    # llama.cpp's blocks (IQ3_S: a grid, signs and a scale a 32; Q4_K: the minimums against the sums of 16), their
    # tables made on the device from a codebooks row
    tables = arena.alloc(34992)
    assert pkg.load_kernels().sb_tables(tables, arena.put(bm.codebooks(rng))) == 34992
    for t in (21, 12):
        blocks = bm.random_blocks(rng, t, rows * (n // 256))
        specs.append(("matmul_sbr", arena.put(blocks), tables, t))
    x = rng.standard_normal((tokens, n)).astype(F)
    return arena.put(x), specs


def run_both(pkg, arena, ax, specs, n, tokens, rows):
    """hq_matmuls with the caller's a / b (a frame of 2n a token), then hq_matmuls_static (a = b = 0 in the table);
    returns both outputs of every job"""
    from pyodide_llm_amd import jobs
    L = pkg.library()
    os_ = 4 * rows
    frame = 2 * n
    given, static = [], []
    outs_given, outs_static = [], []
    for kind, wq, ws, wc in specs:
        og = arena.alloc(os_ * tokens, fill=np.full(rows * tokens, -7, F))
        ost = arena.alloc(os_ * tokens, fill=np.full(rows * tokens, -9, F))
        ab = arena.alloc(tokens * frame)  # this job's own a / b: hq_matmuls readies into it
        given.append(jobs.job(kind, og, ab, ab + n, wq, ws, wc, n, rows=rows, count=tokens, os=os_, as_=frame,
                              bs=frame))
        static.append(jobs.job(kind, ost, 0, 0, wq, ws, wc, n, rows=rows, count=tokens, os=os_))
        outs_given.append(og)
        outs_static.append(ost)
    assert jobs.matmuls(L, ax, 4 * n, given) == 0, L.hq_last_error_message()
    t = jobs.table(static)
    assert L.hq_matmuls_static(ax, 4 * n, t, len(static), jobs.JOB, None) == 0, L.hq_last_error_message()
    return ([arena.get(o, F, rows * tokens) for o in outs_given], [arena.get(o, F, rows * tokens) for o in outs_static])


def test_static_staging_is_hq_matmuls(pkg, arena, oracle):
    rng = np.random.default_rng(77)
    # a prompt (the matrix-core tiles; the plain kind in slices of four tokens), then a smaller decode
    for n, tokens, rows in ((2048, 20, 200), (1024, 3, 70)):
        arena.reset()
        ax, specs = phase_of(pkg, arena, oracle, rng, n, tokens, rows)
        want, got = run_both(pkg, arena, ax, specs, n, tokens, rows)
        for (kind, _, _, wc), w, g in zip(specs, want, got):
            assert same_bits(g, w), f"n {n} tokens {tokens} {kind} a6 {wc}: {first_difference(g, w)}"
        # and the first job against the oracle, so that the two agreeing is not two wrong numbers
        x = arena.get(ax, F, tokens * n).reshape(tokens, n)
        w8 = arena.get(specs[0][1], np.int8, rows * n)
        ws = arena.get(specs[0][2], F, rows * n // 32)
        for t in (0, tokens - 1):
            q, s = oracle.quantize_x(x[t], 64)
            ref = oracle.matmul_q8r(q, s, w8, ws, oracle.int8_sums(w8), n)
            assert same_bits(got[0][t * rows:(t + 1) * rows], ref), f"n {n} token {t}"


def test_static_staging_refuses_what_does_not_fit(pkg):
    from pyodide_llm_amd import jobs
    L = pkg.library()
    n = 4096
    fits = STAGING // staged_frame(n)
    job = jobs.job("matmul_q8r", 4096, 0, 0, 4096, 4096, 0, n, rows=8, count=fits + 1, os=32)
    assert L.hq_matmuls_static(4096, 4 * n, jobs.table([job]), 1, jobs.JOB, None) == pkg.HQ_ERR_ARGUMENT
    assert "staging" in L.hq_last_error_message().decode()
    L.hq_clear_error()


def test_static_staging_under_graph_capture(pkg, arena, oracle):
    """the callers it is for: hq_matmuls_static captured into a HIP graph (no allocation, no memset in it), replayed
    three times with new inputs written eagerly between the replays, each replay's outputs checked against an eager
    hq_matmuls of the same inputs"""
    import torch
    from pyodide_llm_amd import jobs
    L = pkg.library()
    assert L.hq_init() == 0
    rng = np.random.default_rng(78)
    n, tokens, rows = 1024, 2, 96
    arena.reset()
    ax, specs = phase_of(pkg, arena, oracle, rng, n, tokens, rows)
    os_ = 4 * rows
    outs = [arena.alloc(os_ * tokens) for _ in specs]
    table = jobs.table([jobs.job(kind, o, 0, 0, wq, ws, wc, n, rows=rows, count=tokens, os=os_)
                        for (kind, wq, ws, wc), o in zip(specs, outs)])
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        h = stream.cuda_stream
        assert L.hq_matmuls_static(ax, 4 * n, table, len(specs), jobs.JOB, h) == 0, L.hq_last_error_message()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            L.hq_matmuls_static(ax, 4 * n, table, len(specs), jobs.JOB, h)
    assert L.hq_last_error() == 0, L.hq_last_error_message()
    for replay in range(3):
        x = rng.standard_normal((tokens, n)).astype(F) * (replay + 1)
        arena.write(ax, x)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [arena.get(o, F, rows * tokens) for o in outs]
        want, _ = run_both(pkg, arena, ax, specs, n, tokens, rows)
        for (kind, _, _, wc), w_, g_ in zip(specs, want, got):
            assert same_bits(g_, w_), f"replay {replay} {kind} wc {bool(wc)}: {first_difference(g_, w_)}"
