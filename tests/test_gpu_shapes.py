"""The benchmark configs' shapes at full size (stories15M, LFM2-350M, Llama-3.2-1B, Llama-3-8B, the 27B-class low-bit
matrices), through the C-ABI on cuda:0, bit for bit against the oracle: every row of the token products, and for
the prompts (M = 256 .. 2048 tokens) every row of a sample of tokens spread over the token tiles, plus a property
that holds at any size (tokens that are copies of each other give the same outputs, wherever their tiles are)."""
import numpy as np
import pytest

from gpu_util import Arena, first_difference, same_bits
from models import F
from streams import pack6

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def k(pkg):
    import torch
    assert torch.cuda.is_available(), "the GPU tests need a GPU"
    return pkg.load_kernels()


@pytest.fixture(scope="module")
def arena():
    return Arena(3 << 29)


@pytest.fixture(autouse=True)
def fresh(arena):
    arena.reset()
    yield


def int8_matrix(rng, rows, n):
    """the configs' weights: int8 uniform in [-127, 127], scales |N(0, 0.02)| / 127 a group of 32"""
    w = rng.integers(-127, 128, rows * n, dtype=np.int8)
    ws = (np.abs(rng.standard_normal(rows * n // 32)) * (0.02 / 127)).astype(F)
    return w, ws


def prompt(oracle, rng, count, n, bias=64, copies=()):
    """count tokens of N(0, 1) activations quantized per token, in frames; tokens in `copies` (pairs) duplicated"""
    frame = ((n + 4 * (n // 32) + 15) // 16) * 16
    buf = np.zeros((count, frame), np.uint8)
    for t in range(count):
        q, s = oracle.quantize_x(rng.standard_normal(n).astype(F), bias)
        buf[t, :n] = q
        buf[t, n:n + 4 * (n // 32)] = s.view(np.uint8)
    for a, b in copies:
        buf[b] = buf[a]
    return buf, frame


@pytest.mark.parametrize("name,rows,n", [("stories15M", 768, 288), ("LFM2 qkv", 1536, 1024),
                                         ("LFM2 gate+up", 9216, 1024), ("LFM2 down", 1024, 4608),
                                         ("LFM2 lm-head", 65536, 1024), ("8B qkv", 6144, 4096),
                                         ("8B down", 4096, 14336), ("8B lm-head", 128256, 4096)])
def test_decode_q8r_full(k, arena, oracle, name, rows, n):
    """M = 1 and M = 4 (one launch reads the weights once for the 4 tokens): every row, int8_sums' wc and wc NULL"""
    rng = np.random.default_rng(rows + n)
    w, ws = int8_matrix(rng, rows, n)
    wc = oracle.int8_sums(w)
    buf, frame = prompt(oracle, rng, 4, n)
    wq, wsa, wca, xq = arena.put(w), arena.put(ws), arena.put(wc), arena.put(buf)
    want = [oracle.matmul_q8r(buf[t, :n], buf[t, n:n + 4 * (n // 32)].view(F), w, ws, wc, n) for t in range(4)]
    for c in (wca, 0):
        out = arena.alloc(4 * rows)
        k.matmul_q8r(out, xq, xq + n, wq, wsa, c, n, 0, rows)
        got = arena.get(out, F, rows)
        assert same_bits(got, want[0]), f"{name} M=1 wc {bool(c)}: {first_difference(got, want[0])}"
        out4 = arena.alloc(4 * rows * 4)
        k.matmul_q8r_tile(out4, xq, xq + n, wq, wsa, c, n, 0, rows, 4, 4 * rows, frame)
        got4 = arena.get(out4, F, rows * 4).reshape(4, rows)
        for t in range(4):
            assert same_bits(got4[t], want[t]), f"{name} M=4 token {t}: {first_difference(got4[t], want[t])}"


SAMPLE = [0, 1, 31, 32, 63, 64, 100, 255]


@pytest.mark.parametrize("name,rows,n,count", [("1B qkv", 3072, 2048, 512), ("1B o", 2048, 2048, 512),
                                               ("1B gate", 8192, 2048, 512), ("1B down", 2048, 8192, 512),
                                               ("8B gate", 14336, 4096, 2048), ("8B down", 4096, 14336, 2048)])
def test_prefill_q8r_tile(k, arena, oracle, name, rows, n, count):
    rng = np.random.default_rng(rows * 7 + n)
    w, ws = int8_matrix(rng, rows, n)
    wc = oracle.int8_sums(w)
    copies = [(3, count - 1), (5, count // 2 + 17)]
    buf, frame = prompt(oracle, rng, count, n, copies=copies)
    wq, wsa, wca, xq = arena.put(w), arena.put(ws), arena.put(wc), arena.put(buf)
    sample = sorted({t for t in SAMPLE + [count - 1, count - 64, count // 2] if t < count})
    for c in (wca, 0):
        out = arena.alloc(4 * rows * count)
        k.matmul_q8r_tile(out, xq, xq + n, wq, wsa, c, n, 0, rows, count, 4 * rows, frame)
        got = arena.get(out, F, rows * count).reshape(count, rows)
        for t in sample:
            want = oracle.matmul_q8r(buf[t, :n], buf[t, n:n + 4 * (n // 32)].view(F), w, ws, wc, n)
            assert same_bits(got[t], want), f"{name} token {t} wc {bool(c)}: {first_difference(got[t], want)}"
        for a, b in copies:
            assert same_bits(got[a], got[b]), f"{name}: tokens {a} and {b} are the same, their outputs are not"


@pytest.mark.parametrize("rows,n", [(17408, 5120), (5120, 17408)])
def test_27b_int6(pkg, k, arena, oracle, rows, n):
    """config 4(b): int6 weights v uniform in [-31, 31] (stored 4 v, scale / 4), M = 1 every row, M = 256 sampled"""
    from pyodide_llm_amd import jobs
    rng = np.random.default_rng(rows + 6)
    v = (4 * rng.integers(-31, 32, rows * n)).astype(np.int8)
    packed = pack6(v)
    ws = (np.abs(rng.standard_normal(rows * n // 32)) * (0.02 / 31 / 4)).astype(F)
    wc = oracle.six_sums(packed)
    count = 256
    buf, frame = prompt(oracle, rng, count, n, copies=[(2, 250)])
    wq, wsa, wca, xq = arena.put(packed), arena.put(ws), arena.put(wc), arena.put(buf)
    want0 = oracle.matmul_q6r(buf[0, :n], buf[0, n:n + 4 * (n // 32)].view(F), packed, ws, wc, n)
    out = arena.alloc(4 * rows)
    k.matmul_q6r(out, xq, xq + n, wq, wsa, wca, n, 0, rows)
    got = arena.get(out, F, rows)
    assert same_bits(got, want0), first_difference(got, want0)
    outs = arena.alloc(4 * rows * count)
    job = jobs.job("matmul_q6r", outs, xq, xq + n, wq, wsa, wca, n, rows=rows, count=count, os=4 * rows, as_=frame,
                   bs=frame)
    assert jobs.phase(pkg.library(), [job]) == 0, pkg.library().hq_last_error_message()
    got = arena.get(outs, F, rows * count).reshape(count, rows)
    for t in (0, 1, 33, 64, 127, 200, 255):
        want = oracle.matmul_q6r(buf[t, :n], buf[t, n:n + 4 * (n // 32)].view(F), packed, ws, wc, n)
        assert same_bits(got[t], want), f"token {t}: {first_difference(got[t], want)}"
    assert same_bits(got[2], got[250])


@pytest.mark.parametrize("rows,n", [(17408, 5120), (5120, 17408)])
def test_27b_ternary(k, arena, oracle, rows, n):
    """config 4(a): ternary codes with P(0) = 1/3, one float16 scale a row replicated into its groups of 128 (the
    reference's layout), activations quantize_x(bias 0) + interleave; M = 1 every row, M = 256 sampled"""
    from streams import pack_ternary
    rng = np.random.default_rng(rows + 3)
    codes = rng.integers(0, 3, rows * n).astype(np.uint8)
    wq_bytes = pack_ternary(codes)
    row_scale = (np.abs(rng.standard_normal(rows)) * 0.02 + 1e-3).astype(np.float16)
    ws_bits = np.repeat(row_scale, n // 128).view(np.uint16)
    count = 256
    frame = ((n + 8 * (n // 32) + 15) // 16) * 16
    buf = np.zeros((count, frame), np.uint8)
    for t in range(count):
        q, s = oracle.quantize_x(rng.standard_normal(n).astype(F), 0)
        a, area = oracle.interleave(q.view(np.int8), s)
        buf[t, :n] = a.view(np.uint8)
        buf[t, n:n + 8 * (n // 32)] = area.view(np.uint8)
    buf[200] = buf[7]
    wq, wsa, xq = arena.put(wq_bytes), arena.put(ws_bits), arena.put(buf)
    area0 = buf[0, n:n + 8 * (n // 32)].view(F)
    want0 = oracle.matmul_t2r(buf[0, :n].view(np.int8), area0, wq_bytes, ws_bits, n)
    out = arena.alloc(4 * rows)
    k.matmul_t2r(out, xq, xq + n, wq, wsa, n, 0, rows, 3)
    got = arena.get(out, F, rows)
    assert same_bits(got, want0), first_difference(got, want0)
    outs = arena.alloc(4 * rows * count)
    k.matmul_t2r_tile(outs, xq, xq + n, wq, wsa, n, 0, rows, count, 4 * rows, frame, 3)
    got = arena.get(outs, F, rows * count).reshape(count, rows)
    for t in (0, 1, 31, 32, 63, 64, 128, 255):
        want = oracle.matmul_t2r(buf[t, :n].view(np.int8), buf[t, n:n + 8 * (n // 32)].view(F), wq_bytes, ws_bits, n)
        assert same_bits(got[t], want), f"token {t}: {first_difference(got[t], want)}"
    assert same_bits(got[7], got[200])
