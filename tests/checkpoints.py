"""Synthetic llama2.c checkpoints for the loader's tests, written from the format as llama2.c and the reference's
quantize.py lay it out (not from the loader's placement): the header's 7 int32, then the tensors of a Llama in
llama2.c's order — the embedding, every layer's attention norm, then q, k, v and o of every layer, the FFN norms,
w1, w2 and w3 of every layer, the final norm, the RoPE tables (float files only) and the classifier where the
vocabulary is negative.  A float file holds every tensor as float32 / float16; a quantized one every matrix as its
values then its scales, and the norms as float32 (src/python/engine/dtypes.py, packing.py).

write(header, dtype, rng) -> (the file's bytes, {name: (offset of the values, offset of the scales or None, size)})
"""
import struct

import numpy as np

from streams import pack6, pack_binary, pack_ternary


def shapes(header):
    dim, hidden, layers, heads, kv_heads, vocab, seq = header
    head = dim // heads
    q, kv = heads * head, kv_heads * head
    out = [("token_embedding_table", "m", (abs(vocab), dim)), ("rms_att_weight", "v", (layers, dim)),
           ("wq", "m", (layers, q, dim)), ("wk", "m", (layers, kv, dim)), ("wv", "m", (layers, kv, dim)),
           ("wo", "m", (layers, dim, q)), ("rms_ffn_weight", "v", (layers, dim)),
           ("w1", "m", (layers, hidden, dim)), ("w2", "m", (layers, dim, hidden)), ("w3", "m", (layers, hidden, dim)),
           ("rms_final_weight", "v", (dim,)), ("freq_cis_real", "t", (seq, head // 2)),
           ("freq_cis_imag", "t", (seq, head // 2))]
    return out if vocab > 0 else out + [("wcls", "m", (abs(vocab), dim))]


def int8_group(length):
    g = 32
    while length % g:
        g //= 2
    return g


def packed(dtype, count, length, rng):
    """(the values' bytes, the scales' bytes) of a matrix of count weights in rows of length"""
    if dtype == "int8":
        g = int8_group(length)
        v = rng.integers(-127, 128, count).astype(np.int8)
        return v.tobytes(), (rng.random(count // g).astype(np.float32) * 0.01).tobytes()
    if dtype == "int6":
        v = (4 * rng.integers(-31, 32, count)).astype(np.int8)
        return pack6(v).tobytes(), (rng.random(count // 32).astype(np.float32) * 0.01).tobytes()
    if dtype == "ternary":
        codes = rng.integers(0, 3, count).astype(np.uint8)
        return pack_ternary(codes).tobytes(), (rng.random(count // 128) * 0.01 + 1e-3).astype(np.float16).tobytes()
    if dtype == "binary":
        bits = rng.integers(0, 2, count).astype(np.uint8)
        return pack_binary(bits, length).tobytes(), (rng.random(count // 128) * 0.01 + 1e-3).astype(np.float16).tobytes()
    raise ValueError(dtype)


def write(header, dtype, rng, final_norm=None):
    """a checkpoint of this header and dtype with random weights; final_norm: the final norm's weights (default
    random, no outliers)"""
    parts, where, at = [struct.pack("<7i", *header)], {}, 28
    for name, role, shape in shapes(header):
        count = int(np.prod(shape))
        if dtype in ("float32", "float16"):
            data = (rng.standard_normal(count) * 0.02).astype(dtype).tobytes()
            where[name] = (at, None, len(data))
            parts.append(data)
            at += len(data)
            continue
        if role == "t":
            continue  # a quantized file has no RoPE tables
        if role == "v":
            v = rng.random(count).astype(np.float32) + 0.5
            if name == "rms_final_weight" and final_norm is not None:
                v = np.asarray(final_norm, np.float32)
            data = v.tobytes()
            where[name] = (at, None, len(data))
            parts.append(data)
            at += len(data)
            continue
        values, scales = packed(dtype, count, shape[-1], rng)
        where[name] = (at, at + len(values), len(values) + len(scales))
        parts += [values, scales]
        at += len(values) + len(scales)
    return b"".join(parts), where
