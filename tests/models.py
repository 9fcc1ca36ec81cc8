"""The reference tests' own models of the kernels (tests/int8-check.ts:51-90, tests/ternary-check.ts:129-139), written
in NumPy float32 step by step, and the crafted inputs the order-revealing tests use.  Test-side helpers only: they
check the oracle, they are not the oracle."""
import numpy as np

from streams import uninterleave_index

F = np.float32


def nearest(v):
    """tests/int8-check.ts:51-54: round half to even."""
    return np.rint(v)


def quantize_x_model(x, bias):
    """tests/int8-check.ts:248-257, group by group: s = f(largest / qmax), inv = s > 0 ? f(1 / s) : 0, the value
    nearest(f(x inv)) truncated with saturation (NaN -> 0), the bias added in int32 (wrapping), then clamped to int8."""
    x = np.asarray(x, F)
    qmax = F(127.0) if bias == 0 else F(63.0)
    xq = np.zeros(x.size, np.uint8)
    xs = np.zeros(x.size // 32, F)
    for g in range(x.size // 32):
        group = x[g * 32:(g + 1) * 32]
        largest = F(0.0)
        for v in group:
            largest = max(largest, abs(v))
        with np.errstate(all="ignore"):
            s = F(largest / qmax)
            inv = F(F(1.0) / s) if s > 0 else F(0.0)
        xs[g] = s
        for j, v in enumerate(group):
            with np.errstate(all="ignore"):
                r = nearest(F(v * inv))
            t = 0 if np.isnan(r) else int(max(-(2.0 ** 31), min(2.0 ** 31 - 1, float(r))))
            q = ((t + bias + 2 ** 31) % 2 ** 32) - 2 ** 31
            q = max(-128, min(127, q))
            xq[g * 32 + j] = q & 255
    return xq, xs


def q8r_model(w, q, ws, xs, ng):
    """tests/int8-check.ts:65-77: one row of matmul_q8r."""
    lanes = [F(0)] * 4
    ng4 = ng & ~3
    w = np.asarray(w, np.int64)
    q = np.asarray(q, np.int64)

    def exact(g):
        return int(np.sum(w[g * 32:g * 32 + 32] * (q[g * 32:g * 32 + 32] - 64)))

    g = 0
    while g < ng4:
        lanes[g & 3] = F(lanes[g & 3] + F(F(exact(g)) * F(ws[g] * xs[g])))
        g += 1
    s = F(F(F(lanes[0] + lanes[1]) + lanes[2]) + lanes[3])
    while g < ng:
        s = F(s + F(F(exact(g)) * F(ws[g] * xs[g])))
        g += 1
    return s


def q8_model(w, q, ws, xs, ng):
    """tests/int8-check.ts:79-90: one row of matmul_q8 (activations -127..127)."""
    lanes = [F(0)] * 4
    w = np.asarray(w, np.int64)
    q = np.asarray(q, np.int64)
    for g in range(ng):
        s = F(ws[g] * xs[g])
        for k in range(4):
            total = 0
            for half in (0, 16):
                for p in (2 * k, 2 * k + 1, 2 * k + 8, 2 * k + 9):
                    total += int(w[g * 32 + half + p] * q[g * 32 + half + p])
            lanes[k] = F(lanes[k] + F(F(total) * s))
    return F(F(F(lanes[0] + lanes[1]) + lanes[2]) + lanes[3])


def t2_model(codes_row, a, xs, d, groups):
    """tests/ternary-check.ts:129-139: one row of matmul_t2r / matmul_t2; codes_row the row's codes (0..3) in weight
    order, a the activations before interleave(), xs their scales, d the row's group scales as float32."""
    lanes = [F(0)] * 4
    codes_row = np.asarray(codes_row, np.int64)
    a = np.asarray(a, np.int64)
    for g in range(groups):
        for lane in range(4):
            j0 = g * 128 + lane * 32
            total = int(np.sum((codes_row[j0:j0 + 32] - 1) * a[j0:j0 + 32]))
            lanes[lane] = F(lanes[lane] + F(F(F(total) * xs[g * 4 + lane]) * d[g]))
    return F(F(F(lanes[0] + lanes[1]) + lanes[2]) + lanes[3])


def interleave_model(a):
    """tests/ternary-check.ts:95-103: the bytes and sums interleave() must leave."""
    a = np.asarray(a, np.int8)
    n = a.size
    permuted = a[uninterleave_index(n)]
    sums = -a.astype(np.int64).reshape(-1, 32).sum(axis=1)
    return permuted, sums.astype(np.int32)


# ---- crafted inputs: one exact integer a group and a power-of-two scale, so that each group's product is known

def crafted_q8r(ds, es, n_extra_zero_rows=0):
    """matmul_q8r inputs for one row whose group g has the integer dot(w, q - 64) = ds[g] and the scale product
    2^es[g] (ws = 2^e, xs = 1): activation 65 at the group's first value and 64 elsewhere, weight ds[g] there."""
    ng = len(ds)
    n = ng * 32
    w = np.zeros((1 + n_extra_zero_rows, n), np.int8)
    xq = np.full(n, 64, np.uint8)
    for g, d in enumerate(ds):
        xq[g * 32] = 65
        w[0, g * 32] = d
    ws = np.zeros((1 + n_extra_zero_rows, ng), F)
    ws[0] = [F(2.0 ** e) for e in es]
    xs = np.ones(ng, F)
    wc = (-64 * w.astype(np.int32).reshape(-1, 32).sum(axis=1)).astype(np.int32)
    return xq, xs, w.reshape(-1), ws.reshape(-1), wc, n
