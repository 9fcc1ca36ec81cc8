"""The C-ABI (include/hq.h) without a GPU: the library loads, exports every declared symbol with the reference
kernels' argument lists, and refuses bad arguments on the host before anything reaches a device."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "hq.h")


def declared():
    """(name, argument count) of every function include/hq.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[\w\s]+?\*?\s*(\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.M):
        name, args = m.group(1), m.group(2).strip()
        out[name] = 0 if args in ("", "void") else len(args.split(","))
    return out


def test_every_declared_symbol_is_exported(pkg):
    lib = pkg.library()
    names = declared()
    assert len(names) >= 30
    for name in names:
        assert hasattr(lib, name), name


def test_reference_names_and_arities(pkg):
    """The reference kernels keep their names and argument counts (src/runtime/jobs.ts:101-140)."""
    names = declared()
    reference = {"quantize_x": 5, "int8_sums": 3, "six_sums": 3, "interleave": 3, "matmul_q8r": 9, "matmul_q8": 8,
                 "matmul_q8r_tile": 12, "matmul_q6r": 9, "matmul_q6": 8, "matmul_t2r": 9, "matmul_t2": 9,
                 "matmul_t2r_tile": 12, "matmul_b1r": 9, "matmul_b1": 9, "matmul_b1r_tile": 12, "binary_x": 4,
                 "quantize6_x": 4, "ternary_x": 4,
                 "sb_tables": 2, "sums_x": 3, "matmul_sbr": 9, "matmul_sb": 9, "matmul_sbr_tile": 12,
                 "matmul_sbw_tile": 13, "signed_dots": 3, "sb_row": 5, "add_columns": 5}
    for name, arity in reference.items():
        assert names[name] == arity, name
        assert len(pkg.REFERENCE_SIGNATURES[name]) == arity, name
    for name, (argtypes, _) in pkg.OWN_SIGNATURES.items():
        assert names[name] == len(argtypes), name


def test_version(pkg):
    assert pkg.library().hq_version().startswith(b"hq ")


@pytest.mark.parametrize("call, code, words", [
    (lambda L: L.hq_matmul_q8r_ex(None, None, None, None, None, None, 33, 0, 1, None), 1, "multiple of 32"),
    (lambda L: L.hq_matmul_q8r_ex(None, None, None, None, None, None, 64, 3, 2, None), 1, "rows 3..2"),
    (lambda L: L.hq_matmul_q8r_ex(None, None, None, None, None, None, 64, 0, 2, None), 3, "NULL"),
    (lambda L: L.hq_matmul_t2r_ex(16, 16, 16, 16, 16, 128, 0, 1, 2, None), 1, "three"),
    (lambda L: L.hq_matmul_t2r_ex(16, 16, 16, 16, 16, 96, 0, 1, 3, None), 1, "multiple of 128"),
    (lambda L: L.hq_matmul_b1r_ex(16, 16, 16, 16, 16, 128, 0, 1, 3, None), 1, "two = 3, not 2"),
    (lambda L: L.hq_matmul_b1r_ex(16, 16, 16, 16, 16, 192, 0, 1, 2, None), 1, "multiple of 128"),
    (lambda L: L.hq_matmul_b1r_tile_ex(16, 16, 16, 16, 16, 128, 0, 1, 2, 4, 8, 2, None), 2, "frame"),
    (lambda L: L.hq_binary_x_ex(16, 16, 16, 100, None, None), 1, "multiple of 128"),
    (lambda L: L.hq_binary_x_ex(16, 16, 8, 128, None, None), 2, "aligned"),
    (lambda L: L.hq_quantize6_x_ex(16, 16, 16, 48, None), 1, "multiple of 32"),
    (lambda L: L.hq_quantize6_x_ex(16, 18, 16, 32, None), 2, "aligned"),
    (lambda L: L.hq_ternary_x_ex(16, 16, 16, 100, None, None), 1, "multiple of 128"),
    (lambda L: L.hq_ternary_x_ex(16, 16, 8, 128, None, None), 2, "aligned"),
    (lambda L: L.hq_matmul_sbr_ex(16, 16, 16, 16, 16, 256, 0, 1, 11, None), 1, "type 11"),
    (lambda L: L.hq_matmul_sbr_ex(16, 16, 16, 16, 16, 384, 0, 1, 12, None), 1, "multiple of 256"),
    (lambda L: L.hq_matmul_sbr_ex(16, 16, 16, 17, 16, 256, 0, 1, 12, None), 2, "w not 2-byte"),
    (lambda L: L.hq_matmul_sbr_ex(16, 16, 16, 16, 8, 256, 0, 1, 12, None), 2, "tables"),
    (lambda L: L.hq_matmul_sbr_ex(16, 16, 8, 16, 16, 256, 0, 1, 12, None), 2, "xq or xs"),
    (lambda L: L.hq_matmul_sbr_tile_ex(16, 16, 16, 16, 16, 256, 0, 1, 2, 4, 8, 12, None), 2, "token stride"),
    (lambda L: L.hq_matmul_sbr_ex(16, 16, 16, 16, 16, 256, 0, 30000000, 12, None), 1, "4 GiB"),
    (lambda L: L.hq_sb_row_ex(16, 16, 16, 100, 16, None), 1, "multiple of 256"),
    (lambda L: L.hq_sums_x_batch(16, 16, 100, 1, 0, None), 1, "multiple of"),
    (lambda L: L.hq_add_columns_ex(16, 16, 16, -1, 8, None), 1, "count = -1"),
    (lambda L: L.hq_add_columns_ex(16, 18, 16, 1, 8, None), 2, "4-byte"),
    (lambda L: L.hq_outlier_columns_ex(16, 16, 16, 4, None, 0, 8, 32, None), 1, "packing 4"),
    (lambda L: L.hq_outlier_columns_ex(16, 16, 16, 2, None, 0, 8, 64, None), 1, "whole groups of 128"),
    (lambda L: L.hq_outlier_columns_ex(16, 16, 16, 0, (ctypes.c_int32 * 1)(32), 1, 8, 32, None), 1, "not below 32"),
    (lambda L: L.hq_outlier_columns_ex(16, 16, 16, 0, (ctypes.c_int32 * 65)(), 65, 8, 32, None), 1, "at most 64"),
    (lambda L: L.hq_take_channels_ex(16, 16, None, 2, None), 3, "channels NULL"),
    (lambda L: L.hq_matmul_q8_ex(16, 17, 16, 16, 16, 64, 0, 1, None), 2, "xq"),
    (lambda L: L.hq_matmul_q6_ex(16, 16, 16, 12, 16, 64, 0, 1, None), 2, "wq"),
    (lambda L: L.hq_matmul_q8r_tile_ex(16, 16, 16, 16, 16, 16, 64, 0, 1, 3, 4, 8, None), 2, "frame"),
    (lambda L: L.hq_matmul_q8r_tile_ex(16, 16, 16, 16, 16, 16, 64, 0, 1, 3, 6, 16, None), 2, "os"),
    (lambda L: L.hq_quantize_x_ex(16, 16, 16, 48, 0, None), 1, "multiple of 32"),
    (lambda L: L.hq_interleave_ex(16, 16, 96, None), 1, "multiple of 64"),
    (lambda L: L.hq_int8_sums_ex(16, 8, 4, None), 2, "aligned"),
])
def test_argument_errors_on_host(pkg, call, code, words):
    L = pkg.library()
    L.hq_clear_error()
    assert call(L) == code
    assert L.hq_last_error() == code
    assert words in L.hq_last_error_message().decode()
    L.hq_clear_error()
    assert L.hq_last_error() == 0


def test_empty_ranges_launch_nothing(pkg):
    """Zero rows or zero tokens: nothing to do, no device needed, no error (the reference's loops run zero times)."""
    L = pkg.library()
    assert L.hq_matmul_q8r_ex(None, None, None, None, None, None, 64, 5, 5, None) == 0
    assert L.hq_matmul_q8r_tile_ex(None, None, None, None, None, None, 64, 0, 9, 0, 0, 0, None) == 0
    assert L.hq_quantize_x_batch(None, None, None, 64, 64, 0, 0, 0, None) == 0


def test_drop_in_records_errors(pkg):
    """The drop-in names return nothing and keep the error for hq_last_error (Kernels raises HQError)."""
    k = pkg.load_kernels()
    with pytest.raises(pkg.HQError) as e:
        k.matmul_q8r(0, 0, 0, 0, 0, 0, 100, 0, 4)
    assert e.value.code == pkg.HQ_ERR_ARGUMENT
    assert pkg.library().hq_last_error() == 0  # cleared once raised


def test_phase_refuses_other_kinds_and_bad_numbers(pkg):
    from pyodide_llm_amd import jobs
    L = pkg.library()
    attention = jobs.job("attention", 16, 16, 16, 16, 16, 0, 64, rows=4)
    assert jobs.phase(L, [attention]) == pkg.HQ_ERR_KIND
    assert "kind 3" in L.hq_last_error_message().decode()
    bad = jobs.job("matmul_q8r", 16.5, 16, 16, 16, 16, 16, 64, rows=4)
    assert jobs.phase(L, [bad]) == pkg.HQ_ERR_ARGUMENT
    odd = jobs.job("matmul_t2r", 16, 16, 16, 16, 16, 0, 100, rows=4)
    assert jobs.phase(L, [odd]) == pkg.HQ_ERR_ARGUMENT
    odd = jobs.job("matmul_b1", 16, 16, 16, 16, 16, 0, 64, rows=4)
    assert jobs.phase(L, [odd]) == pkg.HQ_ERR_ARGUMENT
    untyped = jobs.job("matmul_sbr", 16, 16, 16, 16, 16, 11, 256, rows=4)
    assert jobs.phase(L, [untyped]) == pkg.HQ_ERR_ARGUMENT
    assert "type 11" in L.hq_last_error_message().decode()
    assert jobs.phase(L, []) == 0


def test_work_numbers_match_the_reference():
    """KIND is each kind's place in jobs.ts's WORK (jobs.ts:207-336); hq.h names 0, 1, 5, 6, 8..14."""
    from pyodide_llm_amd import jobs
    assert [jobs.KIND[k] for k in ("matmul_q8r", "matmul_q8", "matmul_q6r", "matmul_q6", "matmul_t2r", "matmul_t2",
                                   "matmul_sbr", "matmul_sb", "matmul_sbw", "matmul_b1r", "matmul_b1")] == \
        [0, 1, 5, 6, 8, 9, 10, 11, 12, 13, 14]
    assert {name: jobs.BLOCK_TYPES[name][0] for name in jobs.BLOCK_TYPES} == \
        {"Q2_K": 10, "Q4_K": 12, "IQ2_XXS": 16, "IQ2_XS": 17, "IQ3_XXS": 18, "IQ1_S": 19, "IQ3_S": 21, "IQ2_S": 22,
         "IQ4_XS": 23, "IQ1_M": 29}
    assert jobs.PACKED["int8"].weight_bytes() == 1.125
    assert jobs.PACKED["int6"].weight_bytes() == 0.875
    assert jobs.PACKED["ternary"].weight_bytes() == 0.265625
    assert jobs.PACKED["binary"].weight_bytes() == 0.140625  # (16 + 2) / 128


def test_job_path_keeps_tile_offsets_in_32_bits(pkg):
    """The matrix-core tiles keep a lane's offsets within a tile of 64 tokens (128 for llama.cpp's blocks) and 128
    rows in 32 bits: a prompt whose activations are 64 MiB apart (or whose rows are 32 MiB long) takes the token
    kernel, which gives the same numbers with 64-bit addresses."""
    from pyodide_llm_amd import jobs
    L = pkg.library()
    q8r, t2r, q8, sbr = (jobs.KIND[k] for k in ("matmul_q8r", "matmul_t2r", "matmul_q8", "matmul_sbr"))
    n = 4096
    frame = n + n // 8
    assert L.hq_job_path(q8r, n, 2048, frame, frame) == 1
    assert L.hq_job_path(q8r, n, 15, frame, frame) == 0  # under 16 tokens: the token kernel
    assert L.hq_job_path(q8, n, 2048, frame, frame) == 0  # no matrix-core tile for the plain form
    big = 1 << 26  # 64 tokens x 64 MiB reach 4 GiB
    assert L.hq_job_path(q8r, n, 2048, big - 4096, big - 4096) == 1
    assert L.hq_job_path(q8r, n, 2048, big, frame) == 0
    assert L.hq_job_path(q8r, n, 2048, frame, big) == 0
    assert L.hq_job_path(t2r, n, 64, big, big) == 0
    assert L.hq_job_path(t2r, n, 64, frame, frame) == 1
    assert L.hq_job_path(q8r, 1 << 25, 64, 1 << 25, 1 << 25) == 0  # 128 rows of 32 MiB
    assert L.hq_job_path(sbr, n, 64, 1 << 24, 4096) == 0  # the blocks' tile: frames under 16 MiB
    assert L.hq_job_path(sbr, n, 64, (1 << 24) - 16, 4096) == 1
    assert L.hq_job_path(3, n, 64, frame, frame) == -1  # attention is not a kind run here


def test_matmuls_refuses_two_frames(pkg):
    """hq_matmuls readies each token's bytes and scales one frame apart (the reference's S): a job whose a and b
    advance by different strides is refused on the host, as are jobs of two inputs."""
    from pyodide_llm_amd import jobs
    L = pkg.library()
    two = jobs.job("matmul_q8", 16, 16, 4096, 16, 16, 0, 64, rows=4, count=2, os=16, as_=256, bs=512)
    assert jobs.matmuls(L, 16, 256, [two]) == pkg.HQ_ERR_ARGUMENT
    assert "one frame" in L.hq_last_error_message().decode()
    a = jobs.job("matmul_q8r", 16, 16, 4096, 16, 16, 16, 64, rows=4)
    b = jobs.job("matmul_q8r", 16, 16, 4096, 16, 16, 16, 128, rows=4)
    assert jobs.matmuls(L, 16, 256, [a, b]) == pkg.HQ_ERR_ARGUMENT
    assert "one input" in L.hq_last_error_message().decode()
    L.hq_clear_error()


def test_matmuls_static_refuses_more_than_its_staging(pkg):
    """hq_matmuls_static stages a token's activations round_up(n, 256) + round_up(n / 2, 256) bytes apart in 4 MiB:
    more tokens are refused on the host, before any device is touched"""
    from pyodide_llm_amd import jobs
    L = pkg.library()
    n = 4096
    fits = (4 << 20) // (4096 + 2048)
    job = jobs.job("matmul_q8r", 4096, 0, 0, 4096, 4096, 0, n, rows=8, count=fits + 1, os=32)
    assert L.hq_matmuls_static(4096, 4 * n, jobs.table([job]), 1, jobs.JOB, None) == pkg.HQ_ERR_ARGUMENT
    assert "staging" in L.hq_last_error_message().decode()
    L.hq_clear_error()


def test_matmuls_passes_over_jobs_of_no_rows(pkg):
    """A job of no rows computes nothing, so hq_matmuls neither checks nor readies its a / b (here 0) and takes no
    part of it in the one-input check: a table of only such jobs succeeds without a device or an input."""
    from pyodide_llm_amd import jobs
    L = pkg.library()
    empty = jobs.job("matmul_q8r", 0, 0, 0, 0, 0, 0, 64, rows=0, count=3, os=0, as_=0, bs=0)
    other = jobs.job("matmul_t2r", 0, 0, 0, 0, 0, 0, 4096, rows=0, count=1)
    assert jobs.matmuls(L, 0, 0, [empty, other]) == 0, L.hq_last_error_message()
    assert L.hq_matmuls_static(0, 0, jobs.table([empty]), 1, jobs.JOB, None) == 0, L.hq_last_error_message()


def test_tolerance_tile_refusals_on_host(pkg):
    """hq_matmul_q8r_tile_tol_ex checks its workspace (size, alignment, NULL) and the job before any device work;
    hq_tol_work_bytes is the float16 activations (2 n a token, to 256 bytes) and the scales (n / 32 groups x the
    tokens to a multiple of 4, 4 bytes each)"""
    L = pkg.library()
    assert L.hq_tol_work_bytes(4096, 2048) == 2 * 4096 * 2048 + 128 * 2048 * 4
    assert L.hq_tol_work_bytes(288, 37) == ((2 * 288 * 37 + 255) // 256) * 256 + 9 * 40 * 4
    assert L.hq_tol_work_bytes(100, 4) == -1 and L.hq_last_error() == pkg.HQ_ERR_ARGUMENT
    n, count, need = 1024, 20, L.hq_tol_work_bytes(1024, 20)
    args = (4096, 8192, 8192 + n, 65536, 1 << 20, n, 0, 64, count, 256, 2048)
    assert L.hq_matmul_q8r_tile_tol_ex(*args, 1 << 24, need - 1, None) == pkg.HQ_ERR_ARGUMENT
    assert "workspace" in L.hq_last_error_message().decode()
    assert L.hq_matmul_q8r_tile_tol_ex(*args, (1 << 24) + 128, need, None) == pkg.HQ_ERR_ALIGNMENT
    assert L.hq_matmul_q8r_tile_tol_ex(*args, None, need, None) == pkg.HQ_ERR_NULL
    assert L.hq_matmul_q8r_tile_tol_ex(4096, 8192, 8192, 65536, 1 << 20, 100, 0, 64, count, 256, 2048,
                                       1 << 24, need, None) == pkg.HQ_ERR_ARGUMENT
    assert L.hq_matmul_q8r_tile_tol_ex(None, None, None, None, None, n, 5, 5, count, 256, 2048, None, 0, None) == 0
    L.hq_clear_error()


def test_tol_min_tiles_setting(pkg):
    """hq_tol_min_tiles: -1 by default (a round of two blocks a compute unit), any count of tiles from 0 (every
    launch takes the tolerance tile), each call returning the setting before it; below -1 refused, nothing changed"""
    L = pkg.library()
    before = L.hq_tol_min_tiles(5)
    try:
        assert before == -1
        assert L.hq_tol_min_tiles(0) == 5
        assert L.hq_tol_min_tiles(-2) == pkg.HQ_ERR_ARGUMENT
        assert L.hq_last_error() == pkg.HQ_ERR_ARGUMENT
        L.hq_clear_error()
        assert L.hq_tol_min_tiles(-1) == 0
    finally:
        L.hq_tol_min_tiles(before)


def test_ceiling_epilogue_refusals_on_host(pkg):
    """hq_ceiling_epilogue takes form 0 (the bit-exact tile's epilogue) or 1 (the tolerance tile's), a positive grid
    and iteration count, and an aligned sink, checked before any device work"""
    L = pkg.library()
    assert L.hq_ceiling_epilogue(2, 8, 8, 4096, None) == pkg.HQ_ERR_ARGUMENT
    assert L.hq_ceiling_epilogue(-1, 8, 8, 4096, None) == pkg.HQ_ERR_ARGUMENT
    assert L.hq_ceiling_epilogue(0, 0, 8, 4096, None) == pkg.HQ_ERR_ARGUMENT
    assert L.hq_ceiling_epilogue(1, 8, 0, 4096, None) == pkg.HQ_ERR_ARGUMENT
    assert L.hq_ceiling_epilogue(0, 8, 8, None, None) == pkg.HQ_ERR_NULL
    assert L.hq_ceiling_epilogue(0, 8, 8, 4098, None) == pkg.HQ_ERR_NULL
    L.hq_clear_error()
