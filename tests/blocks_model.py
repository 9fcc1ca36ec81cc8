"""A NumPy model of llama.cpp's blocks of 256 weights, as the reference's converter reads them
(src/python/convert/superblocks.py:56-200, the forms of ggml's block_* structs), for the parity tests of the oracle's
and the GPU's block kernels.  Written from those forms, not from the kernels (kernels/blocks/types.ts), so that a
mistake in the kernels' own unpacking shows as a difference:

  read_ints(type, blocks, grids)   -> per weight: W (its own small integer, signed), S (its unit's integer), M (the
                                      K types' minimum of its unit), and per block F, Fm (the kernels' arithmetic,
                                      types.ts:32-57: a weight is F S W - Fm M)
  read_floats(type, blocks, grids) -> the reader's float32 weights (superblocks.py's order of float32 products)
  matmul(type, blocks, a, xs, grids) -> a row's product in the kernels' float32 order (types.ts:48-57)

The codebooks are a test's own (the kernels take the caller's row of codebooks; these are random grids of the
magnitudes each type allows, types.ts:32-43), in the row's layout: the six grids a value a byte, then IQ4_XS's 16.
"""
import numpy as np

F32 = np.float32
TYPES = {"Q2_K": 10, "Q4_K": 12, "IQ2_XXS": 16, "IQ2_XS": 17, "IQ3_XXS": 18, "IQ1_S": 19, "IQ3_S": 21,
         "IQ2_S": 22, "IQ4_XS": 23, "IQ1_M": 29}
BYTES = {10: 84, 12: 144, 16: 66, 17: 74, 18: 98, 19: 50, 21: 110, 22: 82, 23: 136, 29: 56}
# the grids' places in the codebooks row and their shapes (entries, values an entry)
GRIDS = {"IQ2XXS": (0, 256, 8), "IQ2XS": (2048, 512, 8), "IQ2S": (6144, 1024, 8), "IQ3XXS": (14336, 256, 4),
         "IQ3S": (15360, 512, 4), "IQ1S": (17408, 2048, 8)}
ROW_BYTES = 33792 + 16
# the 7-bit sign indices' eighth sign: the number of minus signs is even
SEVEN = np.array([i | ((bin(i).count("1") & 1) << 7) for i in range(128)], np.uint16)


def codebooks(rng):
    """a row of codebooks: IQ2's magnitudes 8, 25, 43; IQ3_XXS's 4, 12, .., 62; IQ3_S's 1, 3, .., 15; IQ1's -1, 0,
    1; IQ4_XS's 16 values from -127 to 113 (the first and last at the ends)"""
    row = np.zeros(ROW_BYTES, np.uint8)
    two = rng.choice(np.array([8, 25, 43], np.uint8), 2048 + 4096 + 8192)
    row[:14336] = two
    row[14336:15360] = rng.choice(np.arange(4, 63, 8, dtype=np.uint8), 1024)
    row[15360:17408] = rng.choice(np.arange(1, 16, 2, dtype=np.uint8), 2048)
    row[17408:33792] = rng.choice(np.array([-1, 0, 1], np.int8), 16384).view(np.uint8)
    values = np.sort(rng.choice(np.arange(-126, 113), 14, replace=False))
    row[33792:] = np.concatenate([[-127], values, [113]]).astype(np.int8).view(np.uint8)
    return row


def grids(row):
    g = {name: row[at:at + n * k].reshape(n, k).astype(np.int32) for name, (at, n, k) in GRIDS.items()}
    g["IQ1S"] = row[17408:33792].view(np.int8).reshape(2048, 8).astype(np.int32)
    g["IQ4NL"] = row[33792:].view(np.int8).astype(np.int32)
    return g


def ieee_half(bits):
    """float16 bits -> float32 as NumPy (and the converter, superblocks.py:34-36) widen them: infinities and NaNs kept"""
    return np.asarray(bits).astype("<u2").view("<f2").astype(F32)


def kernel_half(bits):
    """float16 bits -> float32 as the kernels widen a block's scales (kernels/blocks/row.ts:3-15 through
    kernels/kernel/halves.ts:20-23): the half sign-extended, shifted left 13, ANDed with 0x8fffffff, as a float32,
    times 2^112 (one float32 product).  Exact for every finite half; an infinity reads as 65536 and a NaN as a finite
    number."""
    b = np.asarray(bits).astype(np.int64) & 0xFFFF
    extended = (b ^ 0x8000) - 0x8000
    moved = ((extended << 13) & 0x8FFFFFFF).astype(np.uint32).view(F32)
    return (moved * F32(2.0 ** 112)).astype(F32)


HALF = ieee_half  # how read_ints widens a block's float16 scales (tests set kernel_half to model the kernels)


def halves(raw):
    return HALF(np.ascontiguousarray(raw).view("<u2").reshape(-1))


def u16(raw):
    return np.ascontiguousarray(raw).view("<u2").astype(np.int64)


def u32(raw):
    return np.ascontiguousarray(raw).view("<u4").astype(np.int64)


def bits_of(byte):
    """(..) bytes -> (.., 8) their bits, the lowest first"""
    return (np.asarray(byte, np.int64)[..., None] >> np.arange(8)) & 1


def read_ints(t, b, g):
    """blocks b (N, bytes) of type t -> W, S, M (N, 256) int64; F, Fm, d (N,) float32 (d: the block's float16 or
    IQ1_M's put together; F = d times the type's power of two)"""
    N = len(b)
    M = np.zeros((N, 256), np.int64)
    Fm = np.zeros(N, F32)
    if t == 10:  # Q2_K: scales[16] qs[64] d dmin; bits 2s, 2s+1 of byte c of half h's 32 are weight 128h + 32s + c
        q = (b[:, 16:80].reshape(N, 2, 1, 32).astype(np.int64) >> (2 * np.arange(4)).reshape(1, 1, 4, 1)) & 3
        W = q.reshape(N, 256)
        unit = np.repeat(b[:, :16].astype(np.int64), 16, axis=1)
        S, M = unit & 15, unit >> 4
        d, Fm = halves(b[:, 80:82]), halves(b[:, 82:84])
        F = d
    elif t == 12:  # Q4_K: d dmin scales[12] qs[128]: six-bit scales and minima of eight groups of 32
        s = b[:, 4:16].astype(np.int64)
        sc = np.concatenate([s[:, :4] & 63, (s[:, 8:] & 15) | ((s[:, :4] >> 6) << 4)], axis=1)
        mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
        q = b[:, 16:].reshape(N, 4, 32).astype(np.int64)
        W = np.stack([q & 15, q >> 4], axis=2).reshape(N, 256)
        S, M = np.repeat(sc, 32, axis=1), np.repeat(mn, 32, axis=1)
        d, Fm = halves(b[:, :2]), halves(b[:, 2:4])
        F = d
    elif t in (16, 18):  # IQ2_XXS / IQ3_XXS: grid indices, and a word a 32: four 7-bit sign indices and s on top
        if t == 16:
            idx = b[:, 2:].reshape(N, 8, 8)[:, :, :4].astype(np.int64)  # (N, 8 groups, 4 entries of 8)
            aux = u32(b[:, 2:].reshape(N, 8, 8)[:, :, 4:].copy()).reshape(N, 8)
            mag = g["IQ2XXS"][idx].reshape(N, 8, 32)
        else:
            idx = b[:, 2:66].reshape(N, 8, 8).astype(np.int64)  # 8 entries of 4 a group
            aux = u32(b[:, 66:98].copy()).reshape(N, 8)
            mag = g["IQ3XXS"][idx].reshape(N, 8, 32)
        signs = SEVEN[(aux[:, :, None] >> (7 * np.arange(4))) & 127]  # (N, 8, 4) bytes of signs
        minus = bits_of(signs).reshape(N, 8, 32)
        W = np.where(minus == 1, -mag, mag).reshape(N, 256)
        S = np.repeat(2 * (aux >> 28) + 1, 32, axis=1)
        d = halves(b[:, :2])
        F = d * F32(0.125 if t == 16 else 0.25)
    elif t == 17:  # IQ2_XS: d, 32 words (9 bits of index, 7 of signs), scales[8]: a nibble a 16
        w = u16(b[:, 2:66].copy()).reshape(N, 32)
        mag = g["IQ2XS"][w & 511].reshape(N, 256)
        minus = bits_of(SEVEN[w >> 9]).reshape(N, 256)
        W = np.where(minus == 1, -mag, mag)
        s = np.stack([b[:, 66:74] & 15, b[:, 66:74] >> 4], axis=2).reshape(N, 16).astype(np.int64)
        S = np.repeat(2 * s + 1, 16, axis=1)
        d = halves(b[:, :2])
        F = d * F32(0.125)
    elif t == 22:  # IQ2_S: d qs[32] signs[32] qh[8] scales[8]: a 10-bit index (2 bits a qh byte's pair), a sign byte
        high = (b[:, 66:74, None].astype(np.int64) >> (2 * np.arange(4))) & 3
        index = b[:, 2:34].astype(np.int64) | (high.reshape(N, 32) << 8)
        mag = g["IQ2S"][index].reshape(N, 256)
        minus = bits_of(b[:, 34:66]).reshape(N, 256)
        W = np.where(minus == 1, -mag, mag)
        s = np.stack([b[:, 74:82] & 15, b[:, 74:82] >> 4], axis=2).reshape(N, 16).astype(np.int64)
        S = np.repeat(2 * s + 1, 16, axis=1)
        d = halves(b[:, :2])
        F = d * F32(0.125)
    elif t == 21:  # IQ3_S: d qs[64] qh[8] signs[32] scales[4]: a 9-bit index (bit k of its 32's qh byte)
        high = (b[:, 66:74, None].astype(np.int64) >> np.arange(8)) & 1
        index = b[:, 2:66].astype(np.int64) | (high.reshape(N, 64) << 8)
        mag = g["IQ3S"][index].reshape(N, 256)
        minus = bits_of(b[:, 74:106]).reshape(N, 256)
        W = np.where(minus == 1, -mag, mag)
        s = np.stack([b[:, 106:110] & 15, b[:, 106:110] >> 4], axis=2).reshape(N, 8).astype(np.int64)
        S = np.repeat(2 * s + 1, 32, axis=1)
        d = halves(b[:, :2])
        F = d
    elif t == 19:  # IQ1_S: d qs[32] 8 words: 11-bit indices (3 bits each from the word), s in bits 12-14, shift in 15
        qh = u16(b[:, 34:50].copy()).reshape(N, 8)
        index = b[:, 2:34].reshape(N, 8, 4).astype(np.int64) | (((qh[:, :, None] >> (3 * np.arange(4))) & 7) << 8)
        grid = g["IQ1S"][index].reshape(N, 8, 32)
        down = (qh >> 15)[:, :, None]
        W = (8 * grid + np.where(down == 1, -1, 1)).reshape(N, 256)
        S = np.repeat(2 * ((qh >> 12) & 7) + 1, 32, axis=1)
        d = halves(b[:, :2])
        F = d * F32(0.125)
    elif t == 29:  # IQ1_M: qs[32] qh[16] 4 words; d the words' top four bits; a nibble of qh a 8 (its top: the shift)
        held = u16(b[:, 48:56].copy()).reshape(N, 4)
        dbits = (held[:, 0] >> 12) | ((held[:, 1] >> 8) & 0xF0) | ((held[:, 2] >> 4) & 0xF00) | (held[:, 3] & 0xF000)
        d = HALF(dbits)
        four = np.stack([b[:, 32:48] & 15, b[:, 32:48] >> 4], axis=2).reshape(N, 32).astype(np.int64)
        index = b[:, :32].astype(np.int64) | ((four & 7) << 8)
        grid = g["IQ1S"][index].reshape(N, 32, 8)
        W = (8 * grid + np.where((four & 8)[:, :, None] != 0, -1, 1)).reshape(N, 256)
        s = ((held[:, :, None] >> (3 * np.arange(4))) & 7).reshape(N, 16)
        S = np.repeat(2 * s + 1, 16, axis=1)
        F = d * F32(0.125)
    elif t == 23:  # IQ4_XS: d scales_h scales_l[4] qs[128]: six-bit scales ls - 32, IQ4NL's values
        high = (u16(b[:, 2:4].copy()).reshape(N, 1) >> (2 * np.arange(8))) & 3
        low = np.stack([b[:, 4:8] & 15, b[:, 4:8] >> 4], axis=2).reshape(N, 8).astype(np.int64)
        S = np.repeat((low | (high << 4)) - 32, 32, axis=1)
        q = b[:, 8:].reshape(N, 8, 16).astype(np.int64)
        W = g["IQ4NL"][np.concatenate([q & 15, q >> 4], axis=2)].reshape(N, 256)
        d = halves(b[:, :2])
        F = d
    else:
        raise ValueError(t)
    return W.astype(np.int64), S.astype(np.int64), M.astype(np.int64), F.astype(F32), Fm.astype(F32), d.astype(F32)


def read_floats(t, b, g):
    """the reader's float32 weights (N, 256), its products in its order: d times the unit's (s + 1/2) / 4 (IQ2),
    (s + 1/2) / 2 (IQ3_XXS) or integer, times W (the grid's value with its sign, IQ1's value plus or minus 1/8),
    less dmin times the minimum for the K types"""
    W, S, M, F, Fm, d = read_ints(t, b, g)
    d = d[:, None]
    if t in (16, 17, 22):
        scale = d * (F32(0.5) + ((S - 1) // 2).astype(F32)) * F32(0.25)
    elif t == 18:
        scale = d * (F32(0.5) + ((S - 1) // 2).astype(F32)) * F32(0.5)
    else:
        scale = d * S.astype(F32)
    if t in (19, 29):  # W = 8 g + 1 or 8 g - 1: the grid's g plus or minus an eighth
        down = (W % 8) == 7
        grid = np.where(down, (W + 1) // 8, (W - 1) // 8)
        v = grid.astype(F32) + np.where(down, F32(-0.125), F32(0.125))
    else:
        v = W.astype(F32)
    out = (scale * v).astype(F32)
    if t in (10, 12):
        out = out - (Fm[:, None] * M.astype(F32))
    return out.astype(F32)


def matmul(t, b, a, xs, g):
    """one row (its blocks b, (n/256, bytes)) times int8 activations a (n) with scales xs (n/32), in the kernels'
    order: per block G[k] = sum of S W a over group k (exact), lane k += f(f(f(G[k] xs[k]) + f(G[k+4] xs[k+4])) F),
    less f(f(f(M[k] xs[k]) + f(M[k+4] xs[k+4])) Fm) for the K types; ((l0 + l1) + l2) + l3"""
    W, S, M, F, Fm, _ = read_ints(t, b, g)
    a = np.asarray(a, np.int64).reshape(-1, 8, 32)
    xs = np.asarray(xs, F32).reshape(-1, 8)
    G = (S * W).reshape(-1, 8, 32)
    Gk = (G * a).sum(2)
    Mk = (M.reshape(-1, 8, 32) * a).sum(2)
    lane = np.zeros(4, F32)
    for blk in range(len(b)):
        for k in range(4):
            lo = F32(F32(Gk[blk, k]) * xs[blk, k])
            hi = F32(F32(Gk[blk, k + 4]) * xs[blk, k + 4])
            part = F32(F32(lo + hi) * F[blk])
            if t in (10, 12):
                mlo = F32(F32(Mk[blk, k]) * xs[blk, k])
                mhi = F32(F32(Mk[blk, k + 4]) * xs[blk, k + 4])
                part = F32(part - F32(F32(mlo + mhi) * Fm[blk]))
            lane[k] = F32(lane[k] + part)
    return F32(F32(F32(lane[0] + lane[1]) + lane[2]) + lane[3])


def random_blocks(rng, t, count, tiny=False):
    """count random blocks of type t, their float16 scales set to sane values (a file's are finite): d in [1e-4, 1e-2]
    (or, tiny, subnormal halves), the K types' dmin likewise"""
    size = BYTES[t]
    b = rng.integers(0, 256, (count, size), dtype=np.uint8)

    def put_half(col, values):
        b[:, col:col + 2] = values.astype("<f2").view(np.uint8).reshape(count, 2)

    def some():
        if tiny:
            return (rng.integers(1, 1024, count) * 2.0 ** -24).astype(np.float16)
        return (rng.random(count) * 1e-2 + 1e-4).astype(np.float16)
    if t == 10:
        put_half(80, some())
        put_half(82, some())
    elif t == 12:
        put_half(0, some())
        put_half(2, some())
    elif t == 29:  # d in the top nibbles of the four words at 48..55
        bits = some().view(np.uint16).astype(np.int64)
        for k in range(4):
            word = u16(b[:, 48 + 2 * k:50 + 2 * k].copy()).reshape(count)
            word = (word & 0x0FFF) | (((bits >> (4 * k)) & 15) << 12)
            b[:, 48 + 2 * k:50 + 2 * k] = word.astype("<u2").view(np.uint8).reshape(count, 2)
    else:
        put_half(0, some())
    return b
