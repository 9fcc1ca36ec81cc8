"""llama2.c checkpoints with their matrices resident in HBM, for the products of libhq.so.

A llama2.c file is a header of seven little-endian int32 (dim, hidden_dim, layers, heads, kv_heads, vocab, seq_len;
a negative vocab: the classifier is a tensor of its own) and then the tensors of a Llama back to back, in the order
llama2.c writes them.  Nothing in the file says how the tensors are stored: the reference tells the storage by the
file's size alone (src/python/engine/checkpoint.py:133-173), each storage fixing every tensor's bytes
(src/python/engine/layout.py:245-730, dtypes.py:37-85).  This module computes the same thing its own way: a table of
spans, one per stored tensor, laid down by a cursor from the bytes per weight of the storage, and the storage found
as the one whose table ends exactly at the file's last byte.  The formats it reads are the reference's:
  float32 / float16   every tensor, RoPE tables included, in that float format;
  int8                matrices as int8 values then a float32 scale a group (a group: the largest power of two up to 32
                      that divides the row), norms as float32, no RoPE tables;
  int6                24 bytes a group of 32, then a float32 scale a group;
  ternary / binary    32 / 16 bytes a group of 128, then a float16 scale a group.
A packed storage (int6, ternary, binary) is possible only where every packed row is whole groups and every packed
tensor ends on a 4-byte boundary (where the next one starts).

The device side follows the forward pass's view of a matrix (src/runtime/forward/tensors.ts:104-143): the packed
values and scales go to HBM once, as the file has them (the kernels read the reference's layouts in place), the
relaxed kinds' corrections are made there by int8_sums / six_sums, `Matrix.layer(l)` gives a layer's device
addresses and `Matrix.job()` its job for `hq_phase` / `hq_matmuls` (jobs.ts:36-46).

The classifier's outlier channels (plan.py:176-183, tensors.ts:170-187, engine.ts:459-466): `outlier_channels` picks
them from the final norm's weight (the reference's rule: the 8 largest |weights|, when the largest is at least 4 times
the median), `Checkpoint` widens their columns of the classifier on the device (hq_outlier_columns_ex) and
`Checkpoint.classify` runs the classifier of one token as the engine does: the channels taken apart, quantize_x and
the product (hq_matmuls), then add_columns.
"""
import math
from typing import NamedTuple, Optional

import numpy as np

HEADER_BYTES = 28
OUTLIER_CHANNELS = 8     # the reference's count and ratio (checkpoint.py:43-44)
OUTLIER_RATIO = 4.0

# what a tensor is, for the storage rules: a norm (float32 in a packed file), a RoPE table (absent from a packed file),
# or a matrix (the embedding and the classifier are matrices here)
NORM, ROPE, MATRIX = "norm", "rope", "matrix"


class Storage(NamedTuple):
    """bits a weight; for a grouped storage the bytes of a group's scale and the group's size for a row length"""
    name: str
    bits: int
    scale_bytes: int = 0
    group_of: Optional[object] = None

    @property
    def grouped(self):
        return self.group_of is not None


def int8_group(length):
    """the largest power of two that divides the row, at most 32 (its lowest set bit)"""
    return min(32, length & -length)


STORAGES = {s.name: s for s in (
    Storage("float32", 32), Storage("float16", 16),
    Storage("int8", 8, 4, int8_group), Storage("int6", 6, 4, lambda length: 32),
    Storage("ternary", 2, 2, lambda length: 128), Storage("binary", 1, 2, lambda length: 128))}
# the storages tried in turn: a size two of them share is the earlier's.  The reference's table of sizes
# (src/python/engine/checkpoint.py:159-169) takes the unpacked storages in the order float32, float16, int8, a later
# one taking over a size an earlier one had, then the packed ones only where a size is still free: int8, float16,
# float32, then int6, ternary, binary.
PREFERENCE = ("int8", "float16", "float32", "int6", "ternary", "binary")
QUANTIZED = ("int8", "int6", "ternary", "binary")


class Shape(NamedTuple):
    dim: int
    hidden_dim: int
    layers: int
    heads: int
    kv_heads: int
    vocab: int
    seq_len: int
    shared_classifier: bool

    @property
    def head_size(self):
        return self.dim // self.heads


def read_header(ints):
    """the header's seven ints as a Shape; ValueError naming the first field that no llama2.c model can have"""
    dim, hidden, layers, heads, kv_heads, vocab, seq_len = (int(v) for v in ints)
    big = 1 << 24
    bounds = (("dim", dim, big), ("hidden_dim", hidden, big), ("layers", layers, 4096), ("heads", heads, big),
              ("kv_heads", kv_heads, big), ("|vocab|", abs(vocab), big), ("seq_len", seq_len, big))
    for field, value, top in bounds:
        if not 0 < value < top:
            raise ValueError(f"refused: header field {field} = {value} is outside 1..{top - 1}")
    if dim % heads:
        raise ValueError(f"refused: header heads = {heads} does not divide dim = {dim}")
    if heads % kv_heads:
        raise ValueError(f"refused: header kv_heads = {kv_heads} does not divide heads = {heads}")
    return Shape(dim, hidden, layers, heads, kv_heads, abs(vocab), seq_len, vocab > 0)


def llama_tensors(shape):
    """(name, what, dims) of every tensor of a llama2.c Llama, in file order: the embedding; per-layer stacks of the
    attention norm, q, k, v, o, the FFN norm, w1 (gate), w2 (down), w3 (up); the final norm; the two RoPE tables;
    the classifier when it is not the embedding"""
    s = shape
    L, hs = s.layers, s.head_size
    q, kv = s.heads * hs, s.kv_heads * hs
    out = [("token_embedding_table", MATRIX, (s.vocab, s.dim)), ("rms_att_weight", NORM, (L, s.dim)),
           ("wq", MATRIX, (L, q, s.dim)), ("wk", MATRIX, (L, kv, s.dim)), ("wv", MATRIX, (L, kv, s.dim)),
           ("wo", MATRIX, (L, s.dim, q)), ("rms_ffn_weight", NORM, (L, s.dim)),
           ("w1", MATRIX, (L, s.hidden_dim, s.dim)), ("w2", MATRIX, (L, s.dim, s.hidden_dim)),
           ("w3", MATRIX, (L, s.hidden_dim, s.dim)), ("rms_final_weight", NORM, (s.dim,)),
           ("freq_cis_real", ROPE, (s.seq_len, hs // 2)), ("freq_cis_imag", ROPE, (s.seq_len, hs // 2))]
    if not s.shared_classifier:
        out.append(("wcls", MATRIX, (s.vocab, s.dim)))
    return out


class Span(NamedTuple):
    """a stored tensor: its bytes [at, end), the values first and, for a grouped storage, the scales from `scales`"""
    name: str
    what: str
    dims: tuple
    storage: str
    at: int
    end: int
    scales: int = 0
    group: int = 0

    @property
    def size(self):
        return self.end - self.at


def spans(shape, storage):
    """the table of a file of this shape in this storage: one Span per stored tensor, back to back from the header's
    end (a packed file keeps its norms float32 and has no RoPE tables); None when the storage cannot hold a row"""
    table, cursor = [], HEADER_BYTES
    packed = storage in QUANTIZED
    for name, what, dims in llama_tensors(shape):
        if packed and what == ROPE:
            continue
        kind = STORAGES["float32" if packed and what == NORM else storage]
        weights = math.prod(dims)
        if not kind.grouped:
            span = Span(name, what, dims, kind.name, cursor, cursor + weights * kind.bits // 8)
        else:
            group = kind.group_of(dims[-1])
            if dims[-1] % group:
                return None
            values = weights * kind.bits // 8
            span = Span(name, what, dims, kind.name, cursor,
                        cursor + values + weights // group * kind.scale_bytes, cursor + values, group)
            if kind.name != "int8" and span.size % 4:
                return None  # a packed tensor ends where the next one starts, on 4 bytes
        table.append(span)
        cursor = span.end
    return table


def file_bytes(shape, storage):
    """the size of a file of this shape in this storage, or None when the storage cannot hold it"""
    table = spans(shape, storage)
    return None if table is None else table[-1].end


def storage_of(shape, size):
    """the storage whose table ends at the file's last byte; ValueError listing what each storage would need"""
    for name in PREFERENCE:
        if file_bytes(shape, name) == size:
            return name
    need = ", ".join(f"{name} {file_bytes(shape, name)}" for name in PREFERENCE if file_bytes(shape, name))
    raise ValueError(f"refused: a file of {size} bytes is no storage of this header (bytes each would take: {need})")


def outlier_channels(weight, count=OUTLIER_CHANNELS, ratio=OUTLIER_RATIO):
    """the `count` channels of the largest |weight| (ties: the lower channel), in channel order; none when the largest
    |weight| is below `ratio` times the median"""
    size = np.abs(np.asarray(weight, dtype=np.float32)).reshape(-1)
    if size.size == 0 or size.max() < ratio * np.median(size):
        return np.zeros(0, dtype=np.intp)
    ranked = np.lexsort((np.arange(size.size), -size))
    return np.sort(ranked[:count])


# the job kinds of a storage (jobs.ts:396-440: relaxed, plain) and the kernel that makes the relaxed corrections
JOB_KINDS = {"int8": ("matmul_q8r", "matmul_q8", "int8_sums"), "int6": ("matmul_q6r", "matmul_q6", "six_sums"),
             "ternary": ("matmul_t2r", "matmul_t2", None), "binary": ("matmul_b1r", "matmul_b1", None)}


class Matrix:
    """A matrix (or a stack of one for each layer) of a quantized checkpoint on the device (tensors.ts:104-143): its
    values and scales as the file has them, the relaxed kinds' corrections made once on the device.  layer(l) ->
    (values, scales, corrections or 0) device addresses of layer l; job() the job of a layer for hq_phase."""

    def __init__(self, torch, lib, check, span, raw, device, relaxed):
        self.name, self.kind, self.group = span.name, span.storage, span.group
        dims = span.dims
        self.layers = dims[0] if len(dims) == 3 else 1
        self.rows, self.n = dims[-2], dims[-1]
        values = span.scales - span.at
        scale_bytes = span.end - span.scales
        groups = math.prod(dims) // span.group
        # one allocation: values, then scales, then corrections (each from a 256-byte boundary)
        scales_at = -(-values // 256) * 256
        sums_at = -(-(scales_at + scale_bytes) // 256) * 256
        relaxed_kind, plain_kind, sums = JOB_KINDS[self.kind]
        # (the int8 kernels take groups of 32: a row of smaller groups runs the plain kind, without corrections)
        relaxed = relaxed and span.group in (32, 128)
        self.job_kind = relaxed_kind if relaxed else plain_kind
        with_sums = relaxed and sums is not None
        self.memory = torch.empty(sums_at + (4 * groups if with_sums else 0), dtype=torch.uint8, device=device)
        self.memory[:values].copy_(torch.from_numpy(np.array(raw[span.at:span.scales])))
        self.memory[scales_at:scales_at + scale_bytes].copy_(torch.from_numpy(np.array(raw[span.scales:span.end])))
        base = self.memory.data_ptr()
        self.values, self.scales = base, base + scales_at
        self.corrections = 0
        if with_sums:
            self.corrections = base + sums_at
            check(getattr(lib, f"hq_{sums}_ex")(self.corrections, self.values, groups, None))
        self.row_bytes = values // (self.layers * self.rows)
        self.layer_scales = scale_bytes // self.layers
        self.layer_sums = 4 * (groups // self.layers)

    def layer(self, l):
        """tensors.ts:130-133: layer l's values, scales and corrections (0: none)"""
        if not 0 <= l < self.layers:
            raise IndexError(f"{self.name} has {self.layers} layers, not {l + 1}")
        return (self.values + l * self.rows * self.row_bytes, self.scales + l * self.layer_scales,
                self.corrections and self.corrections + l * self.layer_sums)

    def job(self, l, out, xq, xs, count=1, os=0, frame=0, rows=None):
        """layer l's job (jobs.ts:36-46) for `count` tokens at xq / xs (a frame apart) into out (os apart): a6 the
        corrections (0 where the kind has none)"""
        from . import jobs
        wq, ws, wc = self.layer(l)
        return jobs.job(self.job_kind, out, xq, xs, wq, ws, wc, self.n, rows=self.rows if rows is None else rows,
                        count=count, os=os, as_=frame, bs=frame)


class Checkpoint:
    """A llama2.c checkpoint (a path or the file's bytes) read for the GPU: its shape, the storage its size says, its
    table of spans; the quantized matrices on the device (`matrices`, by name), the float32 norms on the host
    (`vectors`), and for a quantized classifier its outlier channels and their columns on the device."""

    def __init__(self, source, device="cuda:0", relaxed=True):
        import torch

        from . import check, library
        if isinstance(source, (bytes, bytearray, memoryview)):
            raw = np.frombuffer(source, dtype=np.uint8)
        else:
            raw = np.memmap(source, dtype=np.uint8, mode="r")
        if raw.size < HEADER_BYTES:
            raise ValueError(f"refused: {raw.size} bytes hold no 28-byte header")
        self.header = tuple(int(v) for v in raw[:HEADER_BYTES].view("<i4"))
        self.shape = read_header(self.header)
        self.dtype = storage_of(self.shape, raw.size)
        if self.dtype not in QUANTIZED:
            raise ValueError(f"refused: libhq multiplies quantized matrices and this file is {self.dtype}")
        self.relaxed = relaxed
        self.spans = {s.name: s for s in spans(self.shape, self.dtype)}
        lib = library()
        self.lib, self.torch, self.device = lib, torch, device
        self.matrices, self.vectors = {}, {}
        for name, span in self.spans.items():
            if span.storage == "float32":
                self.vectors[name] = np.array(raw[span.at:span.end]).view("<f4").reshape(span.dims)
            else:
                self.matrices[name] = Matrix(torch, lib, check, span, raw, device, relaxed)
        self.classifier = self.matrices["wcls" if "wcls" in self.matrices else "token_embedding_table"]
        # plan.py:176-183: the outlier channels of a quantized classifier, at most dim of them
        self.channels = [int(c) for c in outlier_channels(self.vectors["rms_final_weight"],
                                                          min(OUTLIER_CHANNELS, self.shape.dim))]
        self.columns = self.picked = None
        if self.channels:
            from . import HQ_PACK
            import ctypes
            c = self.classifier
            self.columns = torch.empty(len(self.channels), self.shape.vocab, dtype=torch.float32, device=device)
            self.picked = torch.zeros(len(self.channels), dtype=torch.float32, device=device)
            self._channels = (ctypes.c_int32 * len(self.channels))(*self.channels)
            check(lib.hq_outlier_columns_ex(self.columns.data_ptr(), c.values, c.scales, HQ_PACK[c.kind],
                                            self._channels, len(self.channels), self.shape.vocab, self.shape.dim,
                                            None))

    def classify(self, x, logits, xq, stream=None):
        """engine.ts:459-466 for one token on the device: x (the final norm's dim float32 output, device; its outlier
        channels are set to 0 here, as the engine's are) times the classifier into logits (vocab float32), through
        a scratch xq of the caller's (a frame of the classifier's activations: dim + dim / 2 bytes, 16-byte
        aligned).  With outlier channels: taken apart, the product, add_columns."""
        from . import check, jobs
        lib, s_ = self.lib, self.shape
        s = getattr(stream, "cuda_stream", stream)
        if self.channels:
            check(lib.hq_take_channels_ex(self.picked.data_ptr(), x, self._channels, len(self.channels), s))
        job = self.classifier.job(0, logits, xq, xq + s_.dim)
        check(jobs.matmuls(lib, x, 4 * s_.dim, [job], s))
        if self.channels:
            check(lib.hq_add_columns_ex(logits, self.columns.data_ptr(), self.picked.data_ptr(), len(self.channels),
                                        s_.vocab, s))
