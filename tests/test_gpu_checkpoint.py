"""The loader and the classifier's outlier path on the GPU, through the C-ABI: add_columns, the columns' widening and
the channels taken apart bit for bit against the oracle; checkpoints of every quantized dtype written by
tests/checkpoints.py, loaded into HBM by pyodide-llm_amd/checkpoint.py, their bytes and corrections checked, layers'
products through hq_phase and the classifier of a token (outlier channels apart) against the oracle."""
import ctypes

import numpy as np
import pytest

import checkpoints
from gpu_util import Arena, first_difference, same_bits

pytestmark = pytest.mark.gpu
F = np.float32


@pytest.fixture(scope="module")
def arena():
    import torch
    assert torch.cuda.is_available(), "the GPU tests need a GPU"
    return Arena(1 << 26)


@pytest.fixture(autouse=True)
def fresh(arena):
    arena.reset()
    yield


def channel_array(channels):
    return (ctypes.c_int32 * max(1, len(channels)))(*channels)


@pytest.mark.parametrize("n", [1, 3, 255, 256, 257, 50257, 128256])
@pytest.mark.parametrize("count", [0, 1, 8])
def test_add_columns(pkg, arena, oracle, n, count):
    rng = np.random.default_rng(n + count)
    y = rng.standard_normal(n).astype(F) * 4
    rows = rng.standard_normal((max(count, 1), n)).astype(F)[:count]
    a = rng.standard_normal(max(count, 1)).astype(F)[:count] * 9
    want = oracle.add_columns(y, rows, a)
    ay = arena.put(y)
    L = pkg.library()
    assert L.hq_add_columns_ex(ay, arena.put(rows) if count else arena.alloc(4), arena.put(a) if count else
                               arena.alloc(4), count, n, None) == 0
    got = arena.get(ay, F, n)
    assert same_bits(got, want), first_difference(got, want)
    if count:  # the drop-in, once more on the same y
        pkg.load_kernels().add_columns(ay, arena.put(rows), arena.put(a), count, n)
        want2 = oracle.add_columns(want, rows, a)
        assert same_bits(arena.get(ay, F, n), want2)


@pytest.mark.parametrize("packing,dim", [("int8", 288), ("int8", 48), ("int6", 256), ("ternary", 384),
                                         ("binary", 256)])
def test_outlier_columns(pkg, arena, oracle, packing, dim):
    rng = np.random.default_rng(dim)
    vocab = 1001
    if packing == "int8":
        group = checkpoints.int8_group(dim)
        raw = rng.integers(-128, 128, vocab * dim).astype(np.int8).view(np.uint8)
        s = (rng.random(vocab * dim // group) + 0.5).astype(F)
    else:
        group = 32 if packing == "int6" else 128
        raw, s = checkpoints.packed(packing, vocab * dim, dim, rng)
        raw = np.frombuffer(raw, np.uint8)
        s = np.frombuffer(s, F if packing == "int6" else np.uint16)
    channels = [0, 5, dim - 1, dim // 2, 17]
    want = oracle.outlier_columns(packing, raw, s, channels, vocab, dim, group)
    out = arena.alloc(4 * len(channels) * vocab, fill=np.full(len(channels) * vocab, -7, F))
    L = pkg.library()
    assert L.hq_outlier_columns_ex(out, arena.put(raw), arena.put(s), pkg.HQ_PACK[packing], channel_array(channels),
                                   len(channels), vocab, dim, None) == 0, L.hq_last_error_message()
    got = arena.get(out, F, len(channels) * vocab).reshape(len(channels), vocab)
    assert same_bits(got, want), first_difference(got, want)
    # a channel beyond the row is refused, nothing run
    assert L.hq_outlier_columns_ex(out, 16, 16, 0, channel_array([dim]), 1, vocab, dim, None) == pkg.HQ_ERR_ARGUMENT


def test_take_channels(pkg, arena, oracle):
    x = np.random.default_rng(2).standard_normal(4096).astype(F)
    channels = [3, 17, 200, 4095]
    want_p, want_x = oracle.take_channels(x, channels)
    ax, ap = arena.put(x), arena.alloc(4 * len(channels))
    assert pkg.library().hq_take_channels_ex(ap, ax, channel_array(channels), len(channels), None) == 0
    assert same_bits(arena.get(ap, F, len(channels)), want_p)
    assert same_bits(arena.get(ax, F, x.size), want_x)


def file_tensor(data, where, name):
    at, scales, size = where[name]
    raw = np.frombuffer(data, np.uint8)
    return raw[at:scales], raw[scales:at + size]


def activations(oracle, x, packing):
    """the oracle's preparation of x for a packing's relaxed kernels (jobs.ts:376-379, 421-424)"""
    if packing in ("ternary", "binary"):
        q, s = oracle.quantize_x(x, 0)
        return oracle.interleave(q.view(np.int8), s)
    return oracle.quantize_x(x, 64)


def product(oracle, packing, xq, xs, values, scales, n):
    if packing == "int8":
        return oracle.matmul_q8r(xq, xs, values.view(np.int8), scales.view(F), oracle.int8_sums(values.view(np.int8)), n)
    if packing == "int6":
        return oracle.matmul_q6r(xq, xs, values, scales.view(F), oracle.six_sums(values), n)
    if packing == "ternary":
        return oracle.matmul_t2r(xq, xs, values, scales.view(np.uint16), n)
    return oracle.matmul_b1r(xq, xs, values, scales.view(np.uint16), n)


@pytest.mark.parametrize("dtype,header", [
    ("int8", (288, 768, 6, 6, 6, 32000, 256)),       # stories15M's shapes (the shared classifier)
    ("int6", (256, 768, 2, 4, 2, -1000, 64)),
    ("ternary", (256, 768, 2, 4, 4, -1000, 64)),
    ("binary", (384, 1024, 2, 6, 6, 1000, 64))])
def test_loaded_checkpoint(pkg, arena, oracle, tmp_path, dtype, header):
    import torch
    from pyodide_llm_amd import checkpoint, jobs
    rng = np.random.default_rng(header[0])
    dim = header[0]
    norm = rng.random(dim).astype(F) + 0.5
    norm[[1, 50, dim - 3]] = [40.0, -30.0, 25.0]  # three outliers: eight channels taken apart
    data, where = checkpoints.write(header, dtype, rng, final_norm=norm)
    path = tmp_path / f"model.{dtype}"
    path.write_bytes(data)
    ck = checkpoint.Checkpoint(str(path))
    assert ck.dtype == dtype and ck.header == header
    assert ck.channels == sorted(np.argsort(-np.abs(norm))[:8].tolist())
    L = pkg.library()
    packing = dtype
    # the bytes on the device are the file's; the corrections are int8_sums' / six_sums'
    for name in ("wq", "w2", ck.classifier.name):
        m = ck.matrices[name]
        values, scales = file_tensor(data, where, name)
        torch.cuda.synchronize()
        mem = m.memory.cpu().numpy()
        assert np.array_equal(mem[:values.size], values), name
        off = m.scales - m.values
        assert np.array_equal(mem[off:off + scales.size], scales), name
        if m.corrections:
            sums = oracle.int8_sums(values.view(np.int8)) if dtype == "int8" else oracle.six_sums(values)
            off = m.corrections - m.values
            assert np.array_equal(mem[off:off + 4 * sums.size].view(np.int32), sums), name
    # a layer's products through hq_phase: q, k, v of the last layer and its down projection, for one token
    layer = header[2] - 1
    for names, n in ((("wq", "wk", "wv"), dim), (("w2",), header[1])):
        x = rng.standard_normal(n).astype(F)
        xq, xs = activations(oracle, x, packing)
        axq, axs = arena.put(xq), arena.put(xs)
        table, wants = [], []
        for name in names:
            m = ck.matrices[name]
            out = arena.alloc(4 * m.rows, fill=np.full(m.rows, -7, F))
            table.append(m.job(layer, out, axq, axs))
            values, scales = file_tensor(data, where, name)
            lv = values.size // m.layers
            ls = scales.size // m.layers
            wants.append((out, product(oracle, packing, xq, xs, values[layer * lv:(layer + 1) * lv],
                                       scales[layer * ls:(layer + 1) * ls], n), name))
        assert jobs.phase(L, table) == 0, L.hq_last_error_message()
        for out, want, name in wants:
            got = arena.get(out, F, want.size)
            assert same_bits(got, want), f"{dtype} {name}: {first_difference(got, want)}"
    # the classifier of one token: channels apart, the product, add_columns (engine.ts:459-466)
    x = rng.standard_normal(dim).astype(F)
    ax = arena.put(x)
    vocab = abs(header[5])
    logits = arena.alloc(4 * vocab, fill=np.full(vocab, -7, F))
    scratch = arena.alloc(2 * dim + 64)
    ck.classify(ax, logits, scratch)
    picked, rest = oracle.take_channels(x, ck.channels)
    xq, xs = activations(oracle, rest, packing)
    values, scales = file_tensor(data, where, ck.classifier.name)
    want = product(oracle, packing, xq, xs, values, scales, dim)
    group = {"int8": 32, "int6": 32, "ternary": 128, "binary": 128}[packing]
    columns = oracle.outlier_columns(packing, values, scales if packing in ("int8", "int6") else scales.view(np.uint16),
                                     ck.channels, vocab, dim, group)
    want = oracle.add_columns(want, columns, picked)
    got = arena.get(logits, F, vocab)
    assert same_bits(got, want), f"{dtype} classifier: {first_difference(got, want)}"
    assert same_bits(arena.get(ax, F, dim), rest)
