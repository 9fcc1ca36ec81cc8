"""Writes tests/golden/codebooks.npz: the row of codebooks that llama.cpp's i-quantized blocks index (33 808 bytes:
the grids IQ2XXS, IQ2XS, IQ2S, IQ3XXS, IQ3S, IQ1S one after the other, a value a byte, then IQ4_XS's 16 values), as
the reference's converter lays it down (src/python/convert/grids.py:378-387, `codebooks()`; the tables are llama.cpp's
ggml-common.h's).  It is data: the reader tests (test_blocks_digests.py) need the real grids to reproduce the
reference's own digests of what its block readers read (tests/fixtures/superblocks.json "read").

Run in the build container only, where the reference is mounted:

    python tests/golden/make_codebooks.py [/root/reference]

It loads that one file by its path (it imports NumPy alone) and runs its `codebooks()`; nothing else of the reference
is imported or run.
"""
import hashlib
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main(reference="/root/reference"):
    path = os.path.join(reference, "src", "python", "convert", "grids.py")
    spec = importlib.util.spec_from_file_location("reference_grids", path)
    grids = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(grids)
    row, places = grids.codebooks()
    row = np.frombuffer(row, np.uint8).copy()
    assert row.size == 33808, row.size
    where = np.array([places[name] for name in ("IQ2XXS", "IQ2XS", "IQ2S", "IQ3XXS", "IQ3S", "IQ1S", "IQ4NL")],
                     np.int64)
    out = os.path.join(HERE, "codebooks.npz")
    np.savez_compressed(out, row=row, places=where)
    print(f"{out}: {row.size} bytes, sha256 {hashlib.sha256(row.tobytes()).hexdigest()}, places {where.tolist()}")


if __name__ == "__main__":
    main(*sys.argv[1:])
