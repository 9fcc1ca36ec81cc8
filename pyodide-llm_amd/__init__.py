"""pyodide-llm's quantized-matmul hot path on one AMD Instinct MI355X (gfx950).

The kernels live in libhq.so (csrc/, C-ABI in include/hq.h), built in-tree by build.py.  This package is the host
side above that ABI, mirroring the reference's own interface for the path:

  * `load_kernels()` binds the library's exports by the reference kernels' names with the reference's argument
    types (src/python/engine/kernels.py:31-66: usize -> pointer, i32 -> int32, f32 -> float), so that
    `k.matmul_q8r(out, xq, xs, w, ws, wc, n, r0, r1)` reads as the reference tests' calls do; every address is a
    device address.  A call that the library refuses raises HQError (the library keeps the reason).
  * `jobs` mirrors src/runtime/jobs.ts: the kinds of jobs (WORK), the packings (PACKED), their activations'
    preparation (ready), and a phase of jobs run in one call (hq_phase).

There is no CPU fallback: without libhq.so (or without a gfx950 GPU, for the calls that compute) every call
raises.
"""
import ctypes
import os

from . import jobs  # noqa: F401  (the jobs.ts mirror)

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libhq.so")

HQ_OK, HQ_ERR_ARGUMENT, HQ_ERR_ALIGNMENT, HQ_ERR_NULL, HQ_ERR_HIP, HQ_ERR_KIND, HQ_ERR_DEVICE = range(7)
# the packings of hq_outlier_columns_ex (include/hq.h)
HQ_PACK = {"int8": 0, "int6": 1, "ternary": 2, "binary": 3}


class HQError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"libhq error {code}: {message}")
        self.code = code


p, i32, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_float

# the reference's kernels, by name: src/runtime/jobs.ts:101-140 (Arguments), src/python/engine/kernels.py:42-51
REFERENCE_SIGNATURES = {
    "quantize_x": [p, p, p, i32, i32],
    "int8_sums": [p, p, i32],
    "six_sums": [p, p, i32],
    "interleave": [p, p, i32],
    "matmul_q8r": [p, p, p, p, p, p, i32, i32, i32],
    "matmul_q8": [p, p, p, p, p, i32, i32, i32],
    "matmul_q8r_tile": [p, p, p, p, p, p, i32, i32, i32, i32, i32, i32],
    "matmul_q6r": [p, p, p, p, p, p, i32, i32, i32],
    "matmul_q6": [p, p, p, p, p, i32, i32, i32],
    "matmul_t2r": [p, p, p, p, p, i32, i32, i32, i32],
    "matmul_t2": [p, p, p, p, p, i32, i32, i32, i32],
    "matmul_t2r_tile": [p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32],
    "matmul_b1r": [p, p, p, p, p, i32, i32, i32, i32],
    "matmul_b1": [p, p, p, p, p, i32, i32, i32, i32],
    "matmul_b1r_tile": [p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32],
    "binary_x": [p, p, p, i32],
    "quantize6_x": [p, p, p, i32],
    "ternary_x": [p, p, p, i32],
    "sb_tables": [p, p],
    "sums_x": [p, p, i32],
    "matmul_sbr": [p, p, p, p, p, i32, i32, i32, i32],
    "matmul_sb": [p, p, p, p, p, i32, i32, i32, i32],
    "matmul_sbr_tile": [p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32],
    "matmul_sbw_tile": [p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32, p],
    "signed_dots": [p, p, p],
    "sb_row": [p, p, p, i32, i32],
    "add_columns": [p, p, p, i32, i32],
}
# the reference kernels that return a value (the others return nothing)
REFERENCE_RESTYPES = {"binary_x": i32, "ternary_x": i32, "sb_tables": i32}

# the library's own (include/hq.h, second block): name -> (argtypes, restype)
OWN_SIGNATURES = {
    "hq_version": ([], ctypes.c_char_p),
    "hq_init": ([], i32),
    "hq_set_stream": ([p], i32),
    "hq_get_stream": ([], p),
    "hq_synchronize": ([], i32),
    "hq_last_error": ([], i32),
    "hq_last_error_message": ([], ctypes.c_char_p),
    "hq_clear_error": ([], None),
    "hq_quantize_x_ex": ([p, p, p, i32, i32, p], i32),
    "hq_int8_sums_ex": ([p, p, i32, p], i32),
    "hq_six_sums_ex": ([p, p, i32, p], i32),
    "hq_interleave_ex": ([p, p, i32, p], i32),
    "hq_matmul_q8r_ex": ([p, p, p, p, p, p, i32, i32, i32, p], i32),
    "hq_matmul_q8_ex": ([p, p, p, p, p, i32, i32, i32, p], i32),
    "hq_matmul_q8r_tile_ex": ([p, p, p, p, p, p, i32, i32, i32, i32, i32, i32, p], i32),
    "hq_matmul_q6r_ex": ([p, p, p, p, p, p, i32, i32, i32, p], i32),
    "hq_matmul_q6_ex": ([p, p, p, p, p, i32, i32, i32, p], i32),
    "hq_matmul_t2r_ex": ([p, p, p, p, p, i32, i32, i32, i32, p], i32),
    "hq_matmul_t2r_tile_ex": ([p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32, p], i32),
    "hq_matmul_b1r_ex": ([p, p, p, p, p, i32, i32, i32, i32, p], i32),
    "hq_matmul_b1r_tile_ex": ([p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32, p], i32),
    "hq_binary_x_ex": ([p, p, p, i32, p, p], i32),
    "hq_quantize6_x_ex": ([p, p, p, i32, p], i32),
    "hq_ternary_x_ex": ([p, p, p, i32, p, p], i32),
    "hq_sb_tables_ex": ([p, p, p], i32),
    "hq_matmul_sbr_ex": ([p, p, p, p, p, i32, i32, i32, i32, p], i32),
    "hq_matmul_sbr_tile_ex": ([p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32, p], i32),
    "hq_sb_row_ex": ([p, p, p, i32, i32, p], i32),
    "hq_sums_x_batch": ([p, p, i32, i32, i32, p], i32),
    "hq_add_columns_ex": ([p, p, p, i32, i32, p], i32),
    "hq_outlier_columns_ex": ([p, p, p, i32, ctypes.POINTER(i32), i32, i32, i32, p], i32),
    "hq_take_channels_ex": ([p, p, ctypes.POINTER(i32), i32, p], i32),
    "hq_quantize_x_batch": ([p, p, p, i32, i32, i32, i32, i32, p], i32),
    "hq_interleave_batch": ([p, p, i32, i32, i32, p], i32),
    "hq_phase": ([ctypes.POINTER(ctypes.c_double), i32, i32, p], i32),
    "hq_matmuls": ([p, i32, ctypes.POINTER(ctypes.c_double), i32, i32, p], i32),
    "hq_matmuls_static": ([p, i32, ctypes.POINTER(ctypes.c_double), i32, i32, p], i32),
    "hq_job_path": ([i32, i32, i32, ctypes.c_int64, ctypes.c_int64], i32),
    "hq_tol_work_bytes": ([i32, i32], ctypes.c_int64),
    "hq_tol_min_tiles": ([i32], i32),
    "hq_matmul_q8r_tile_tol_ex": ([p, p, p, p, p, i32, i32, i32, i32, i32, i32, p, ctypes.c_int64, p], i32),
    "hq_ceiling_read": ([p, ctypes.c_int64, p, p], i32),
    "hq_ceiling_mfma": ([i32, i32, p, p], i32),
    "hq_ceiling_epilogue": ([i32, i32, i32, p, p], i32),
}

_lib = None


def library(path=None):
    """libhq.so (this package's, or the one HQ_LIBRARY names) as a ctypes library with every export's signature
    set.  Raises when it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    where = path or os.environ.get("HQ_LIBRARY") or LIBRARY
    if not os.path.exists(where):
        raise HQError(HQ_ERR_DEVICE, f"{where} is not built: run `python pyodide-llm_amd/build.py` "
                                     "(or __graft_entry__.build())")
    lib = ctypes.CDLL(where)
    for name, argtypes in REFERENCE_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = argtypes, REFERENCE_RESTYPES.get(name)
    for name, (argtypes, restype) in OWN_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = argtypes, restype
    if path is None:
        _lib = lib
    return lib


def last_error():
    lib = library()
    return lib.hq_last_error(), (lib.hq_last_error_message() or b"").decode()


def check(status=None):
    """Raise HQError for a failed status (or, with none given, for the last failed drop-in call)."""
    code, message = last_error()
    if status is None:
        status = code
    if status:
        library().hq_clear_error()
        raise HQError(status, message)


class Kernels:
    """The reference kernels by name, on device addresses: calling one enqueues it on the library's stream and
    raises HQError when the library refuses it (engine/kernels.py's load_kernels gives the same names)."""

    def __init__(self, lib=None):
        self._lib = lib or library()

    def __getattr__(self, name):
        if name not in REFERENCE_SIGNATURES:
            raise AttributeError(name)
        fn = getattr(self._lib, name)
        lib = self._lib

        def call(*args):
            lib.hq_clear_error()
            result = fn(*args)
            code = lib.hq_last_error()
            if code:
                message = (lib.hq_last_error_message() or b"").decode()
                lib.hq_clear_error()
                raise HQError(code, message)
            return result

        call.__name__ = name
        return call


def load_kernels(path=None):
    """The kernels of libhq.so by the reference's names (the form of src/python/engine/kernels.py:31-66)."""
    return Kernels(library(path))


def synchronize():
    check(library().hq_synchronize())


def set_stream(stream):
    """Enqueue the drop-in calls on `stream` (a torch.cuda.Stream, a raw hipStream_t address, or None)."""
    handle = getattr(stream, "cuda_stream", stream)
    library().hq_set_stream(handle)
