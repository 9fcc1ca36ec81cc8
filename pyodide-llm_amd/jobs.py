"""The job / kernel boundary of the reference (src/runtime/jobs.ts), mirrored for libhq.so.

WORK's kinds keep their numbers (a kind's number is its place in jobs.ts's WORK, jobs.ts:336), so a job table the
reference's forward pass writes (jobs.ts:36-46: [kind, out, a, b, a4, a5, a6, a7, a8, rows, count, os, as, bs, SIZE,
FIRST]) is the one hq_phase() takes.  PACKED gives each weight packing's bytes, the kinds of its jobs, its corrections
kernel and its activations' preparation (jobs.ts:396-444).  Kinds this library does not run (attention, the delta
rule, float32 rows) keep their numbers and are refused by hq_phase.
"""
import ctypes
from dataclasses import dataclass

# jobs.ts:207-333, in order (the number of a kind is its place)
WORK_ORDER = [
    "matmul_q8r", "matmul_q8", "matmul_f32", "attention", "attention_f16", "matmul_q6r", "matmul_q6", "delta_rule",
    "matmul_t2r", "matmul_t2", "matmul_sbr", "matmul_sb", "matmul_sbw", "matmul_b1r", "matmul_b1",
    "attention_capped", "attention_f16_capped",
]
KIND = {name: number for number, name in enumerate(WORK_ORDER)}
# the kinds libhq.so runs, with what WORK says of them: the module (relaxed or plain), whether a tile takes a prompt's
# tokens in one call (for the others every (row, token) is a call of `one`), and the bytes of a row n wide
RUN = {
    "matmul_q8r": dict(relaxed=True, tile=True, row_bytes=lambda n: n),
    "matmul_q8": dict(relaxed=False, tile=False, row_bytes=lambda n: n),
    "matmul_q6r": dict(relaxed=True, tile=False, row_bytes=lambda n: n * 3 // 4),
    "matmul_q6": dict(relaxed=False, tile=False, row_bytes=lambda n: n * 3 // 4),
    "matmul_t2r": dict(relaxed=True, tile=True, row_bytes=lambda n: n // 4),
    "matmul_t2": dict(relaxed=False, tile=False, row_bytes=lambda n: n // 4),
    "matmul_b1r": dict(relaxed=True, tile=True, row_bytes=lambda n: n // 8),
    "matmul_b1": dict(relaxed=False, tile=False, row_bytes=lambda n: n // 8),
    # llama.cpp's blocks: the bytes of a row depend on the block type (BLOCK_TYPES), a job's a6
    "matmul_sbr": dict(relaxed=True, tile=True, row_bytes=None),
    "matmul_sb": dict(relaxed=False, tile=False, row_bytes=None),
    "matmul_sbw": dict(relaxed=True, tile=True, row_bytes=None),
}
# jobs.ts:380-395 and kernels/blocks/types.ts:60-63: a block type's GGUF number and the bytes of its 256 weights
BLOCK_TYPES = {"Q2_K": (10, 84), "Q4_K": (12, 144), "IQ2_XXS": (16, 66), "IQ2_XS": (17, 74), "IQ3_XXS": (18, 98),
               "IQ1_S": (19, 50), "IQ3_S": (21, 110), "IQ2_S": (22, 82), "IQ4_XS": (23, 136), "IQ1_M": (29, 56)}
JOB = 16            # numbers a job in the reference's table (jobs.ts:21)
ROWS, COUNT = 9, 10  # jobs.ts:46
THREE = 3           # jobs.ts:50
TWO = 2             # jobs.ts:52


@dataclass(frozen=True)
class Packing:
    """One line of PACKED (jobs.ts:367-373)."""
    name: str
    group: int          # the weights one scale is of
    scale: int          # the bytes of a group's scale
    relaxed: str        # the kind of its jobs with relaxed SIMD
    plain: str          # and without
    sums: str           # its corrections kernel, or "" (none)
    takes: str          # the form its activations are in ("biased" / "interleaved")
    xs: int             # the bytes a group of 32 activations takes in xs

    def row_bytes(self, n):
        return RUN[self.relaxed]["row_bytes"](n)

    def weight_bytes(self):
        """jobs.ts:448-450: a group's values and its scale, over the group's weights (1.125, 0.875, 0.265625)."""
        return (self.row_bytes(self.group) + self.scale) / self.group

    def bias(self, relaxed):
        """the activations' bias (jobs.ts:375-379): 64 for the relaxed int8 / int6 kernels, else 0"""
        return 64 if (relaxed and self.takes == "biased") else 0


PACKED = {
    "int8": Packing("int8", 32, 4, "matmul_q8r", "matmul_q8", "int8_sums", "biased", 4),
    "int6": Packing("int6", 32, 4, "matmul_q6r", "matmul_q6", "six_sums", "biased", 4),
    "ternary": Packing("ternary", 128, 2, "matmul_t2r", "matmul_t2", "", "interleaved", 8),
    "binary": Packing("binary", 128, 2, "matmul_b1r", "matmul_b1", "", "interleaved", 8),
}


def ready(kernels, packing, relaxed):
    """jobs.ts:376-379, 421-424: the function that prepares n float32 activations at x into xq and xs for the
    packing's kernels (device addresses), through the library's kernels."""
    bias = packing.bias(relaxed)
    if packing.takes == "interleaved":
        def prepare(xq, xs, x, n):
            kernels.quantize_x(xq, xs, x, n, 0)
            kernels.interleave(xq, xs, n)
    else:
        def prepare(xq, xs, x, n):
            kernels.quantize_x(xq, xs, x, n, bias)
    return prepare


def job(kind, out, a, b, a4, a5, a6, a7, a8=0, rows=0, count=1, os=0, as_=0, bs=0):
    """One job of the reference's table (jobs.ts:36-46), its arguments as WORK's `one` of the kind reads them
    (jobs.ts:212, 222, 246, 252, 266, 276): out, xq, xs, wq, ws, wc (or 0), n, -, rows, count, strides."""
    number = KIND[kind] if isinstance(kind, str) else int(kind)
    return [number, out, a, b, a4, a5, a6, a7, a8, rows, count, os, as_, bs, 0, 0]


def table(jobs):
    """The reference's job table (JOB float64 numbers a job) of a list of jobs."""
    out = (ctypes.c_double * (JOB * max(1, len(jobs))))()
    for i, entry in enumerate(jobs):
        for q, value in enumerate(entry[:JOB]):
            out[i * JOB + q] = float(value)
    return out


def phase(lib, jobs, stream=None):
    """Run a phase of jobs (lists of 14..16 numbers) in one call of hq_phase; returns its status."""
    return lib.hq_phase(table(jobs), len(jobs), JOB, getattr(stream, "cuda_stream", stream))


def matmuls(lib, x, x_stride, jobs, stream=None):
    """engine.ts:381-407 (matmulsAlike): the jobs of one float32 input (device address x, token stride in bytes)
    readied and run in one call of hq_matmuls; returns its status."""
    return lib.hq_matmuls(x, x_stride, table(jobs), len(jobs), JOB, getattr(stream, "cuda_stream", stream))
