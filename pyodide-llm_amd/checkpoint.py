"""llama2.c checkpoints with their matrices resident in HBM, for the products of libhq.so.

The reference reads a checkpoint in three places: its layout (src/python/engine/layout.py: the header's 7 ints, the
tensors of a Llama in file order, each quantized tensor's values then its scales, `placed()` at 245-730), what a
file of a given size holds (src/python/engine/checkpoint.py:133-173, `checkpoint_dtype`) and the forward pass's view
of each matrix (src/runtime/forward/tensors.ts:104-143, `held()`: where a layer's values, scales and corrections
are, the corrections of the relaxed kinds made once by `int8_sums` / `six_sums`).  This module is the same for the
Llama layout of llama2.c's files (the architecture of the benchmark's configs, stories15M and the Llama-3 shapes),
in every dtype of engine/dtypes.py: float32, float16, int8, int6, ternary and binary.  The packed matrices go to
the device once, as the file has them (the kernels read the reference's layouts in place); the corrections are made
there; `Matrix.layer(l)` gives a layer's device addresses and `Matrix.job()` its job for `hq_phase` /
`hq_matmuls` (jobs.ts:36-46).

The classifier's outlier channels (checkpoint.py:115-121, plan.py:176-183, tensors.ts:170-187, engine.ts:459-466)
are here too: `outlier_channels` picks them from the final norm's weight, `Checkpoint` widens their columns of the
classifier on the device (hq_outlier_columns_ex), and `Checkpoint.classify` runs the classifier of one token as the
engine does: the channels taken apart, quantize_x and the product (hq_matmuls), then add_columns.
"""
import math
from typing import NamedTuple

import numpy as np

HEADER = 28  # 7 int32 (layout.py:689: the header's 28 bytes, then one tensor after the other)
# a row's role (layout.py): how a quantized file stores it (kind_of, layout.py:658-668)
EMBEDDING, VECTOR, MATRIX, TABLE, CLASSIFIER = "embedding", "vector", "matrix", "table", "classifier"
OUTLIER_CHANNELS = 8     # checkpoint.py:43
OUTLIER_RATIO = 4.0      # checkpoint.py:44


def group32(length):
    """The values of a group of an int8 row of this length (packing.py:32-37): 32, or the largest power of two below
    it that divides the row."""
    size = 32
    while length % size:
        size //= 2
    return size


class Kind(NamedTuple):
    """How a file holds a tensor (dtypes.py:37-66): its values (itemsize bytes each, or bits a value in groups) and,
    for a quantized one, a scale of `scale` bytes a group (4: float32, 2: float16)."""
    name: str
    itemsize: int = 0
    bits: int = 0
    scale: int = 4
    group: object = None

    def stored_bytes(self, count, group):
        """(the bytes of the values, the bytes of the scales) of count values in groups of group (dtypes.py:73-75)"""
        return count // group * (group * self.bits // 8), self.scale * (count // group)

    def suits(self, length):
        return not self.group or length % self.group(length) == 0

    def ends_aligned(self, count, length):
        """dtypes.py:81-85: a tensor ends on 4 bytes (its scales float32 or an even number of float16)"""
        return not self.group or self.scale % 4 == 0 or (count // self.group(length) * self.scale) % 4 == 0


KINDS = {kind.name: kind for kind in (
    Kind("float32", itemsize=4), Kind("float16", itemsize=2),
    Kind("int8", bits=8, group=group32), Kind("int6", bits=6, group=lambda length: 32),
    Kind("ternary", bits=2, scale=2, group=lambda length: 128), Kind("binary", bits=1, scale=2, group=lambda length: 128),
)}
QUANTIZED = ("int8", "int6", "ternary", "binary")
PACKED = ("int6", "ternary", "binary")  # the quantized kinds of fewer than 8 bits (dtypes.py:165)


class Row(NamedTuple):
    name: str
    role: str
    shape: tuple


class Dims(NamedTuple):
    dim: int
    hidden_dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab_size: int
    seq_len: int
    shared: bool
    head_size: int


def dims_of(header):
    """The header's 7 ints (dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len; a negative vocabulary:
    the classifier is a tensor of its own), refused as checkpoint.py:145-152 refuses them when they make no sense."""
    dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len = (int(v) for v in header)
    head_size = dim // n_heads if n_heads and dim % n_heads == 0 else 0
    limit = 1 << 24
    if not (0 < dim < limit and 0 < hidden_dim < limit and 0 < n_layers < 4096 and 0 < n_kv_heads <= n_heads <= dim
            and 0 < abs(vocab_size) < limit and 0 < seq_len < limit and 0 < head_size < limit
            and n_heads % n_kv_heads == 0):
        raise ValueError("This is not a llama2.c checkpoint: the header makes no sense.")
    return Dims(dim, hidden_dim, n_layers, n_heads, n_kv_heads, abs(vocab_size), seq_len, vocab_size > 0, head_size)


def tensor_rows(header):
    """A Llama's tensors in file order (layout.py:342-386: llama2.c's file): the embedding, the attention's norm and
    q, k, v, o, the FFN's norm and w1 (gate), w2 (down), w3 (up), the final norm, the RoPE tables and, when the
    vocabulary is negative, the classifier."""
    d = dims_of(header)
    q_dim, kv_dim, L = d.n_heads * d.head_size, d.n_kv_heads * d.head_size, d.n_layers
    rows = [Row("token_embedding_table", EMBEDDING, (d.vocab_size, d.dim)),
            Row("rms_att_weight", VECTOR, (L, d.dim)),
            Row("wq", MATRIX, (L, q_dim, d.dim)), Row("wk", MATRIX, (L, kv_dim, d.dim)),
            Row("wv", MATRIX, (L, kv_dim, d.dim)), Row("wo", MATRIX, (L, d.dim, q_dim)),
            Row("rms_ffn_weight", VECTOR, (L, d.dim)),
            Row("w1", MATRIX, (L, d.hidden_dim, d.dim)), Row("w2", MATRIX, (L, d.dim, d.hidden_dim)),
            Row("w3", MATRIX, (L, d.hidden_dim, d.dim)),
            Row("rms_final_weight", VECTOR, (d.dim,)),
            Row("freq_cis_real", TABLE, (d.seq_len, d.head_size // 2)),
            Row("freq_cis_imag", TABLE, (d.seq_len, d.head_size // 2))]
    return rows if d.shared else rows + [Row("wcls", CLASSIFIER, (d.vocab_size, d.dim))]


def kind_of(row, dtype):
    """layout.py:658-668: a float file holds every row in its dtype; a quantized one its vectors as float32, no RoPE
    tables (None: left out), and every other row in its dtype."""
    if dtype not in QUANTIZED:
        return dtype
    return "float32" if row.role == VECTOR else None if row.role == TABLE else dtype


class Place(NamedTuple):
    """Where a row is in the file (layout.py:671-686): its kind (None: nowhere), the offset of its values, all its
    bytes, and for a quantized kind its group and the offset of its scales."""
    row: Row
    kind: object
    offset: int
    size: int
    group: int = 0
    scales: int = 0


def placed(rows, dtype, offset=HEADER):
    """layout.py:689-707: a Place for every row, in file order, one tensor after the other from the header's end"""
    places = []
    for row in rows:
        kind, count = kind_of(row, dtype), math.prod(row.shape)
        if kind is None:
            place = Place(row, None, offset, 0)
        elif KINDS[kind].group:
            group = KINDS[kind].group(row.shape[-1])
            values, scales = KINDS[kind].stored_bytes(count, group)
            place = Place(row, kind, offset, values + scales, group, offset + values)
        else:
            place = Place(row, kind, offset, count * KINDS[kind].itemsize)
        places.append(place)
        offset += place.size
    return places


def file_size(rows, dtype):
    return HEADER + sum(place.size for place in placed(rows, dtype))


def suited(rows, dtype):
    """layout.py:715-725: every row of a packed kind is whole groups and ends on 4 bytes"""
    return all(KINDS[p.kind].suits(p.row.shape[-1]) and KINDS[p.kind].ends_aligned(math.prod(p.row.shape),
                                                                                     p.row.shape[-1])
               for p in placed(rows, dtype) if p.kind)


def checkpoint_dtype(header, size):
    """checkpoint.py:133-173: the dtype a file of `size` bytes with this header holds, told by its size alone (the
    float kinds and int8 first, then the packed ones where the rows suit them); ValueError for anything else."""
    rows = tensor_rows(header)
    sizes = {file_size(rows, name): name for name in ("float32", "float16", "int8")}
    for name in PACKED:
        if suited(rows, name):
            sizes.setdefault(file_size(rows, name), name)
    if size not in sizes:
        raise ValueError(f"This is not a llama2.c checkpoint: its header asks for {file_size(rows, 'float32')} bytes as "
                         f"float32, {file_size(rows, 'float16')} as float16 or {file_size(rows, 'int8')} as int8, and "
                         f"the file has {size}.")
    return sizes[size]


def outlier_channels(weight, count=OUTLIER_CHANNELS, ratio=OUTLIER_RATIO):
    """checkpoint.py:115-121: the count channels with the largest |final-norm weight|, in channel order, or none when
    the largest is less than ratio times the median"""
    size = np.abs(np.asarray(weight, dtype=np.float32))
    if size.max() < ratio * np.median(size):
        return np.zeros(0, dtype=np.intp)
    return np.sort(np.argsort(-size)[:count])


# the kinds of the jobs of a packing (jobs.ts:396-440: relaxed, plain), and whether relaxed needs corrections
JOB_KINDS = {"int8": ("matmul_q8r", "matmul_q8", "int8_sums"), "int6": ("matmul_q6r", "matmul_q6", "six_sums"),
             "ternary": ("matmul_t2r", "matmul_t2", None), "binary": ("matmul_b1r", "matmul_b1", None)}


class Matrix:
    """A matrix (or a stack of one for each layer) of a quantized checkpoint on the device (tensors.ts:104-143): its
    values and scales as the file has them, the relaxed kinds' corrections made once on the device.  layer(l) ->
    (values, scales, corrections or 0) device addresses of layer l; job() the job of a layer for hq_phase."""

    def __init__(self, torch, lib, check, place, raw, device, relaxed):
        self.name, self.kind, self.group = place.row.name, place.kind, place.group
        shape = place.row.shape
        self.layers = shape[0] if len(shape) == 3 else 1
        self.rows, self.n = shape[-2], shape[-1]
        values = place.scales - place.offset
        # one allocation: values, then scales, then corrections (each start 256-byte aligned)
        scales_at = (values + 255) // 256 * 256
        scale_bytes = place.size - values
        groups = math.prod(shape) // place.group
        sums_at = (scales_at + scale_bytes + 255) // 256 * 256
        relaxed_kind, plain_kind, sums = JOB_KINDS[self.kind]
        # (the int8 kernels take groups of 32: a row of smaller groups has no job in this library, and no corrections)
        relaxed = relaxed and place.group in (32, 128)
        self.job_kind = relaxed_kind if relaxed else plain_kind
        with_sums = relaxed and sums is not None
        self.memory = torch.empty(sums_at + (4 * groups if with_sums else 0), dtype=torch.uint8, device=device)
        self.memory[:values].copy_(torch.from_numpy(np.array(raw[place.offset:place.scales])))
        self.memory[scales_at:scales_at + scale_bytes].copy_(
            torch.from_numpy(np.array(raw[place.scales:place.offset + place.size])))
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
    """A llama2.c checkpoint (a path or the file's bytes) read for the GPU: the header, the dtype its size says, every
    tensor's place; the quantized matrices on the device (`matrices`, by name), the float32 vectors on the host
    (`vectors`), and for a quantized classifier its outlier channels and their columns on the device."""

    def __init__(self, source, device="cuda:0", relaxed=True):
        import torch

        from . import check, library
        if isinstance(source, (bytes, bytearray, memoryview)):
            raw = np.frombuffer(source, dtype=np.uint8)
        else:
            raw = np.memmap(source, dtype=np.uint8, mode="r")
        if raw.size < HEADER:
            raise ValueError("This is not a llama2.c checkpoint: it is shorter than its header.")
        self.header = tuple(int(v) for v in raw[:HEADER].view("<i4"))
        self.dims = dims_of(self.header)
        self.dtype = checkpoint_dtype(self.header, raw.size)
        if self.dtype not in QUANTIZED:
            raise ValueError(f"libhq multiplies quantized matrices; this checkpoint is {self.dtype}.")
        self.relaxed = relaxed
        self.places = {p.row.name: p for p in placed(tensor_rows(self.header), self.dtype)}
        lib = library()
        self.lib, self.torch, self.device = lib, torch, device
        self.matrices, self.vectors = {}, {}
        for name, place in self.places.items():
            if place.kind is None:
                continue
            if place.kind == "float32":
                self.vectors[name] = np.array(raw[place.offset:place.offset + place.size]).view("<f4").reshape(
                    place.row.shape)
            else:
                self.matrices[name] = Matrix(torch, lib, check, place, raw, device, relaxed)
        self.classifier = self.matrices["wcls" if "wcls" in self.matrices else "token_embedding_table"]
        # plan.py:176-183: the outlier channels of a quantized classifier, at most dim of them
        self.channels = [int(c) for c in outlier_channels(self.vectors["rms_final_weight"],
                                                          min(OUTLIER_CHANNELS, self.dims.dim))]
        self.columns = self.picked = None
        if self.channels:
            from . import HQ_PACK
            import ctypes
            c = self.classifier
            self.columns = torch.empty(len(self.channels), self.dims.vocab_size, dtype=torch.float32, device=device)
            self.picked = torch.zeros(len(self.channels), dtype=torch.float32, device=device)
            self._channels = (ctypes.c_int32 * len(self.channels))(*self.channels)
            check(lib.hq_outlier_columns_ex(self.columns.data_ptr(), c.values, c.scales, HQ_PACK[c.kind],
                                            self._channels, len(self.channels), self.dims.vocab_size, self.dims.dim,
                                            None))

    def classify(self, x, logits, xq, stream=None):
        """engine.ts:459-466 for one token on the device: x (the final norm's dim float32 output, device; its outlier
        channels are set to 0 here, as the engine's are) times the classifier into logits (vocab float32), through
        a scratch xq of the caller's (a frame of the classifier's activations: dim + dim / 2 bytes, 16-byte
        aligned).  With outlier channels: taken apart, the product, add_columns."""
        from . import check, jobs
        lib, d = self.lib, self.dims
        s = getattr(stream, "cuda_stream", stream)
        if self.channels:
            check(lib.hq_take_channels_ex(self.picked.data_ptr(), x, self._channels, len(self.channels), s))
        job = self.classifier.job(0, logits, xq, xq + d.dim)
        check(jobs.matmuls(lib, x, 4 * d.dim, [job], s))
        if self.channels:
            check(lib.hq_add_columns_ex(logits, self.columns.data_ptr(), self.picked.data_ptr(), len(self.channels),
                                        d.vocab_size, s))
