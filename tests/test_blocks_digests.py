"""llama.cpp's block readers pinned to the reference's own golden vectors.

tests/fixtures/superblocks.json ("read", lines 3-14 of the reference) holds, for each of the ten block types, the
SHA-256 of the float32 values the converter's reader (src/python/convert/superblocks.py) gives for 2000 blocks made
of SHAKE-256's bytes of the type's name, every NaN counted as 0 (tests/superblock_cases.py:12-24,
tests/test_superblocks.py:258-268).  The chain checked here and in tests/test_gpu_blocks.py:

  the reference's digests
    = tests/blocks_model.py's reader (IEEE widening of the float16 scales, as the converter's NumPy widens them),
      with llama.cpp's codebooks (tests/golden/codebooks.npz, written by tests/golden/make_codebooks.py)
  the model with the kernels' widening of a half (kernels/kernel/halves.ts:20-23: an infinity reads as 65536, a NaN
  as a finite number; kernels/blocks/row.ts widens a block's scales that way)
    = the oracle's sb_row, bit for bit on all 2000 blocks of every type
    = the HIP sb_row (test_gpu_blocks.py)
so a field misread alike in the model and the oracle now fails against the reference's numbers.  The two widenings
agree on every finite half (all 65 536 are compared); they differ only in blocks whose scale is an infinity or a NaN,
where the kernels and the converter differ in the reference itself.
"""
import hashlib
import os

import numpy as np
import pytest

import blocks_model as bm

HERE = os.path.dirname(os.path.abspath(__file__))
BLOCKS = 2000
# tests/fixtures/superblocks.json:3-14 of the reference
DIGESTS = {
    "Q2_K": "0bb4071faa3b49c291baa4dec5e011fe4ae60136dde93250ffd249690965f2b7",
    "Q4_K": "fde370337a8f0538e104349f7d6c76a4148aa836039c8a6af223717709731bca",
    "IQ2_XXS": "14a5083bb06f7d100d0235e11f616345b3ffe6a9aede396d8d268de5c97f25ca",
    "IQ2_XS": "b6df896c3388d5b082c61b5335036fd5e97f24ffae1c3daaa17a9aaa3ca44333",
    "IQ3_XXS": "7ea1ed68d137d69d1ba62bab28e70c01de79acc4322241cf2026567a6cf48293",
    "IQ1_S": "e093ca33bfba17cd47f774d8fb7c74770e1e78361633184ffc8982bcae921704",
    "IQ3_S": "3b12d0c73a05d29a9f1d0600dc323514094ff66ea8b731aabb55ee84bfa0b554",
    "IQ2_S": "f119c7d7a0087c5a5982f18ae7a52024c38b6dd0e02ee9648e38ac9d7cef0803",
    "IQ4_XS": "d4a60c16a354272f40d0b05cfe1d19047bba288872267d72ccc37891482e5101",
    "IQ1_M": "4107d5bd0edf305a85a841daa0a83be3a0f7de2c9ef8f788d916bca61fa2e5e7",
}


def codebooks():
    """llama.cpp's codebooks row (33 808 bytes) as the converter lays it down"""
    return np.load(os.path.join(HERE, "golden", "codebooks.npz"))["row"]


def shake_blocks(name):
    """tests/superblock_cases.py:12-14: the 2000 blocks of a type, SHAKE-256's bytes of its name"""
    size = bm.BYTES[bm.TYPES[name]]
    return np.frombuffer(hashlib.shake_256(name.encode()).digest(size * BLOCKS), np.uint8).reshape(BLOCKS, size)


def digest(values):
    """tests/superblock_cases.py:17-24: the SHA-256 of the float32 values, little-endian, every NaN as 0"""
    v = np.asarray(values, np.float32).reshape(-1)
    return hashlib.sha256(np.nan_to_num(v, nan=0.0, posinf=np.inf, neginf=-np.inf).astype("<f4").tobytes()).hexdigest()


def model_floats(name, row, half):
    saved = bm.HALF
    bm.HALF = half
    try:
        with np.errstate(all="ignore"):  # some of the float16 scales are infinities and NaNs
            return bm.read_floats(bm.TYPES[name], shake_blocks(name), bm.grids(row)).reshape(-1)
    finally:
        bm.HALF = saved


def test_the_codebooks_fixture():
    """the row's shape as the kernels and the converter read it: six grids (IQ2's magnitudes 8, 25, 43; IQ3_XXS's
    4..62; IQ3_S's odd 1..15; IQ1's -1, 0, 1) and IQ4_XS's 16 values from -127 to 113 (kvalues_iq4nl)"""
    row = codebooks()
    assert row.size == bm.ROW_BYTES == 33808
    assert set(np.unique(row[:14336])) == {8, 25, 43}
    assert set(np.unique(row[14336:15360])) <= set(range(4, 63, 8)) | {62}
    assert set(np.unique(row[15360:17408])) <= set(range(1, 16, 2))
    assert set(np.unique(row[17408:33792].view(np.int8))) == {-1, 0, 1}
    iq4 = row[33792:].view(np.int8)
    assert iq4[0] == -127 and iq4[-1] == 113 and np.all(np.diff(iq4.astype(np.int32)) > 0)


def test_the_two_widenings_agree_on_every_finite_half():
    h = np.arange(65536)
    ieee, kernel = bm.ieee_half(h), bm.kernel_half(h)
    finite = np.isfinite(ieee)
    assert np.array_equal(ieee[finite].view(np.uint32), kernel[finite].view(np.uint32))
    assert list(bm.kernel_half(np.array([0x7C00, 0xFC00]))) == [65536.0, -65536.0]
    assert np.all(np.isfinite(kernel))


@pytest.mark.parametrize("name", sorted(DIGESTS))
def test_model_reads_the_references_digests(name):
    assert digest(model_floats(name, codebooks(), bm.ieee_half)) == DIGESTS[name]


@pytest.mark.parametrize("name", ["IQ2_XXS", "IQ3_S", "IQ1_M", "IQ4_XS"])
def test_a_wrong_table_value_changes_the_digest(name):
    """the digests see the codebooks: one grid entry (or one IQ4_XS value) changed, and the type's digest moves"""
    row = codebooks().copy()
    at = {"IQ2_XXS": 0 + 8 * 17 + 3, "IQ3_S": 15360 + 4 * 100 + 1, "IQ1_M": 17408 + 8 * 1000 + 5,
          "IQ4_XS": 33792 + 7}[name]
    row[at] = np.uint8(row[at] + 2 if name != "IQ1_M" else (row[at] + 1 if row[at] != 1 else 255))
    assert digest(model_floats(name, row, bm.ieee_half)) != DIGESTS[name]


@pytest.mark.parametrize("name", sorted(DIGESTS))
def test_oracle_sb_row_on_the_digests_blocks(oracle, name):
    """the oracle's reader (row.ts) on the digests' 2000 blocks: the model with the kernels' widening to the bit, and,
    where the two widenings give the same values (every block whose scales are finite), the reference's digest"""
    row = codebooks()
    t = bm.TYPES[name]
    blocks = shake_blocks(name)
    got = oracle.sb_row(blocks.reshape(-1), oracle.sb_tables(row), 256 * BLOCKS, t)
    kernel = model_floats(name, row, bm.kernel_half)
    assert np.array_equal(got.view(np.uint32), kernel.view(np.uint32)), name
    ieee = model_floats(name, row, bm.ieee_half)
    same = (np.nan_to_num(ieee, nan=0.0).view(np.uint32) == kernel.view(np.uint32)).reshape(BLOCKS, 256).all(1)
    assert same.mean() > 0.9  # about 6 % of SHAKE's blocks have a scale that is an infinity or a NaN
    spliced = np.where(np.repeat(same, 256), got, ieee)
    assert digest(spliced) == DIGESTS[name]


@pytest.mark.parametrize("name", sorted(DIGESTS))
def test_oracle_matmul_sbr_with_the_real_codebooks(oracle, name):
    """the oracle's product (the kernels' order) against the model's, with llama.cpp's grids, on rows made of the
    digests' blocks whose scales are finite and small enough that no product overflows"""
    row = codebooks()
    t = bm.TYPES[name]
    blocks = shake_blocks(name)
    with np.errstate(all="ignore"):
        _, _, _, F, Fm, d = bm.read_ints(t, blocks, bm.grids(row))
    ok = np.isfinite(d) & np.isfinite(Fm) & (np.abs(d) < 1e3) & (np.abs(Fm) < 1e3)
    nb, rows = 4, 8
    chosen = blocks[np.nonzero(ok)[0][:nb * rows]]
    assert len(chosen) == nb * rows
    n = 256 * nb
    rng = np.random.default_rng(t)
    q, s = oracle.quantize_x(rng.standard_normal(n).astype(np.float32), 0)
    q = q.view(np.int8)
    got = oracle.matmul_sbr(q, oracle.sums_x(q, s), chosen.reshape(-1), oracle.sb_tables(row), n, t)
    for r in range(rows):
        want = bm.matmul(t, chosen[r * nb:(r + 1) * nb], q, s, bm.grids(row))
        assert got[r].view(np.uint32) == np.float32(want).view(np.uint32), (name, r, got[r], want)
