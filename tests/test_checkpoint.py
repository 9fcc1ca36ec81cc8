"""The loader's host side (pyodide-llm_amd/checkpoint.py) and the outlier path's oracle: the llama2.c layout pinned by
the reference's published file sizes and its own tests' cases, placement against an independent writer
(tests/checkpoints.py), the outlier channels as src/python/engine/checkpoint.py:115-121 picks them (the cases of the
reference's tests/test_outliers.py), and add_columns / the columns' widening against closed forms."""
import numpy as np
import pytest

import checkpoints

F = np.float32
STORIES15M = (288, 768, 6, 6, 6, 32000, 256)


@pytest.fixture(scope="module")
def ck(pkg):
    from pyodide_llm_amd import checkpoint
    return checkpoint


def test_published_sizes_of_stories15m(ck):
    """src/models/built.ts:26, 45 (and tests/models-check.ts:183): karpathy/tinyllamas' stories15M is 60816028
    bytes as float32 and 17101468 as the reference's int8"""
    shape = ck.read_header(STORIES15M)
    assert ck.file_bytes(shape, "float32") == 60816028
    assert ck.file_bytes(shape, "int8") == 17101468
    assert ck.storage_of(shape, 60816028) == "float32"
    assert ck.storage_of(shape, 17101468) == "int8"


def test_sizes_follow_the_layout(ck):
    """tests/test_checkpoint_dtype.py:32-36's case, and checkpoint.py:160-167's closed forms: with M values in the
    matrices and V in the vectors a file is 1.125 M + 4 V (int8, groups of 32), 0.875 M + 4 V (int6), 0.265625 M + 4 V
    (ternary), 0.140625 M + 4 V (binary), besides the header"""
    shape = ck.read_header((64, 172, 3, 8, 2, -300, 128))
    floats = sum(int(np.prod(dims)) for _, _, dims in ck.llama_tensors(shape))
    assert ck.storage_of(shape, 28 + 4 * floats) == "float32"
    assert ck.storage_of(ck.read_header([64, 172, 3, 8, 2, -300, 128]), 28 + 2 * floats) == "float16"
    shape = ck.read_header((128, 384, 2, 4, 4, -512, 64))
    tensors = ck.llama_tensors(shape)
    M = sum(int(np.prod(dims)) for _, what, dims in tensors if what == ck.MATRIX)
    V = sum(int(np.prod(dims)) for _, what, dims in tensors if what == ck.NORM)
    for dtype, per in (("int8", 1.125), ("int6", 0.875), ("ternary", 0.265625), ("binary", 0.140625)):
        size = ck.file_bytes(shape, dtype)
        assert size == 28 + per * M + 4 * V, dtype
        assert ck.storage_of(shape, size) == dtype


def test_a_size_two_storages_share_is_the_references_choice(ck):
    """Tiny headers can give two storages one size: here float16 and int8 are both 308 bytes.  The reference's size
    table lets int8 take a size float16 (or float32) had and the packed storages only a free size
    (src/python/engine/checkpoint.py:159-169): int8 wins."""
    shape = ck.read_header((4, 4, 1, 1, 1, 1, 3))
    assert ck.file_bytes(shape, "float16") == ck.file_bytes(shape, "int8") == 308
    assert ck.storage_of(shape, 308) == "int8"
    assert ck.storage_of(shape, ck.file_bytes(shape, "float32")) == "float32"


def test_packed_storages_need_whole_groups_and_aligned_ends(ck):
    """a packed storage holds only rows of whole groups (int6: 32, ternary and binary: 128), and tensors whose bytes
    end on 4 (dtypes.py:81-85: an odd number of float16 scales would leave the next tensor on 2)"""
    assert ck.file_bytes(ck.read_header((96, 256, 1, 4, 4, 256, 16)), "ternary") is None  # rows of 96
    assert ck.file_bytes(ck.read_header((96, 256, 1, 4, 4, 256, 16)), "int6") is not None
    # dim 128, vocab 129: the embedding has 129 float16 scales (258 bytes): not on 4
    assert ck.file_bytes(ck.read_header((128, 256, 1, 4, 4, 129, 16)), "binary") is None
    assert ck.file_bytes(ck.read_header((128, 256, 1, 4, 4, 130, 16)), "binary") is not None
    assert ck.file_bytes(ck.read_header((40, 64, 1, 4, 4, 10, 16)), "int8") is not None  # groups of 8


@pytest.mark.parametrize("size", [0, 27, 1000, 123456789])
def test_a_file_of_another_size_is_refused(ck, size):
    with pytest.raises(ValueError, match="refused: a file of"):
        ck.storage_of(ck.read_header(STORIES15M), size)


@pytest.mark.parametrize("header, field", [((0, 0, 0, 0, 0, 0, 0), "dim"), ((32, 64, 2, 5, 5, 100, 16), "heads"),
                                           ((32, 64, 2, 4, 3, 100, 16), "kv_heads"), ((-32, 64, 2, 4, 4, 100, 16), "dim"),
                                           ((1885434739, 1, 1, 1, 1, 1, 1), "dim"),
                                           ((32, 64, 4096, 4, 4, 100, 16), "layers")])
def test_a_header_that_makes_no_sense_is_refused(ck, header, field):
    """tests/test_checkpoint_dtype.py:74-78's headers, each refused by the field that is wrong"""
    with pytest.raises(ValueError, match=f"refused: header (field )?{field} ="):
        ck.read_header(header)


def test_int8_groups_follow_the_row(ck):
    """packing.py:32-37: 32, or the largest power of two below it that divides the row"""
    assert [ck.int8_group(n) for n in (288, 768, 48, 40, 36, 7)] == [32, 32, 16, 8, 4, 1]


@pytest.mark.parametrize("dtype", ["float32", "float16", "int8", "int6", "ternary", "binary"])
@pytest.mark.parametrize("shared", [True, False])
def test_spans_match_an_independent_writer(ck, dtype, shared):
    header = (128, 384, 2, 4, 2, 256 if shared else -256, 32)
    data, where = checkpoints.write(header, dtype, np.random.default_rng(1))
    shape = ck.read_header(header)
    assert ck.file_bytes(shape, dtype) == len(data)
    assert ck.storage_of(shape, len(data)) == dtype
    table = {s.name: s for s in ck.spans(shape, dtype)}
    assert set(table) == set(where)
    for name, (offset, scales, size) in where.items():
        s = table[name]
        assert (s.at, s.size) == (offset, size), name
        if scales is not None:
            assert s.scales == scales, name


def test_outlier_channels(ck):
    """the reference's tests/test_outliers.py:16-41 cases"""
    rng = np.random.default_rng(0)
    weight = rng.standard_normal(96).astype(F)
    weight[[7, 40, 95]] = [30.0, -25.0, 20.0]
    assert ck.outlier_channels(weight, 3).tolist() == [7, 40, 95]
    assert (ck.OUTLIER_CHANNELS, ck.OUTLIER_RATIO) == (8, 4.0)
    flat = np.ones(64, dtype=F)
    flat[3] = 3.9
    assert ck.outlier_channels(flat).size == 0
    flat[3] = 4.0
    channels = ck.outlier_channels(flat)
    assert channels.size == 8 and 3 in channels.tolist()
    assert ck.outlier_channels(np.array([1, 1, 1, 9], F), min(8, 4)).tolist() == [0, 1, 2, 3]


def test_add_columns_order(oracle):
    """matmul.ts:248-266: from y[j], one rounded product at a time in the order of the rows.  2^24 + 1 + 1 is 2^24 in
    that order (each 1 lost to the rounding) and 2^24 + 2 if the products were summed first; integers are exact"""
    y = np.array([2.0 ** 24, 0.0, 5.0], F)
    rows = np.array([[1, 1, 2], [1, -1, 3]], F)
    a = np.array([1.0, 1.0], F)
    assert oracle.add_columns(y, rows, a).tolist() == [2.0 ** 24, 0.0, 10.0]
    rng = np.random.default_rng(3)
    for n in (1, 3, 4, 7, 1000):
        y = rng.integers(-100, 100, n).astype(F)
        rows = rng.integers(-100, 100, (5, n)).astype(F)
        a = rng.integers(-10, 10, 5).astype(F)
        assert np.array_equal(oracle.add_columns(y, rows, a), y + a @ rows)
    assert np.array_equal(oracle.add_columns(y, rows[:0], a[:0]), y)


@pytest.mark.parametrize("packing", ["int8", "int6", "ternary", "binary"])
def test_outlier_columns_are_the_widened_classifier(oracle, packing):
    """tensors.ts:175-186 against the reference test's widening (test_outliers.py:8-20: the int8 classifier's
    values times their scales, the columns of the channels) and its packings' independent packers"""
    rng = np.random.default_rng(4)
    vocab, dim = 50, 256
    group = {"int8": 32, "int6": 32, "ternary": 128, "binary": 128}[packing]
    if packing in ("int8", "int6"):
        v = rng.integers(-127, 128, (vocab, dim)).astype(np.int8)
        if packing == "int6":
            v = (4 * rng.integers(-32, 32, (vocab, dim))).astype(np.int8)
        raw = v.view(np.uint8) if packing == "int8" else checkpoints.pack6(v.reshape(-1))
        s = (rng.random((vocab, dim // group)) + 0.5).astype(F)
        widened = (v.astype(F).reshape(vocab, dim // group, group) * s[:, :, None]).reshape(vocab, dim)
        raw_s = s
    else:
        codes = rng.integers(0, 3 if packing == "ternary" else 2, (vocab, dim)).astype(np.uint8)
        raw = checkpoints.pack_ternary(codes.reshape(-1)) if packing == "ternary" else checkpoints.pack_binary(
            codes.reshape(-1), dim)
        value = codes.astype(np.int32) - 1 if packing == "ternary" else 2 * codes.astype(np.int32) - 1
        s = (rng.random((vocab, dim // group)) * 0.01 + 1e-3).astype(np.float16)
        widened = (value.astype(F).reshape(vocab, dim // group, group) * s.astype(F)[:, :, None]).reshape(vocab, dim)
        raw_s = s
    channels = [3, 100, 255]
    got = oracle.outlier_columns(packing, raw, raw_s, channels, vocab, dim, group)
    assert got.shape == (3, vocab) and got.dtype == F
    assert np.array_equal(got, widened[:, channels].T), packing


def test_take_channels(oracle):
    x = np.arange(10, dtype=F) + 1
    picked, rest = oracle.take_channels(x, [2, 7])
    assert picked.tolist() == [3.0, 8.0] and rest[2] == 0 and rest[7] == 0 and rest.sum() == x.sum() - 11
