"""Device memory for the GPU tests: one arena (a torch uint8 tensor on cuda:0) that hands out aligned addresses, as
the reference tests place everything in one WebAssembly.Memory (tests/int8-check.ts:121-124)."""
import numpy as np
import torch


class Arena:
    def __init__(self, nbytes):
        self.t = torch.zeros(int(nbytes), dtype=torch.uint8, device="cuda:0")
        self.base = self.t.data_ptr()
        self.top = 0

    def alloc(self, nbytes, align=256, fill=None):
        off = (self.top + align - 1) // align * align
        if off + nbytes > self.t.numel():
            raise MemoryError(f"arena of {self.t.numel()} bytes is full")
        self.top = off + int(nbytes)
        if fill is not None:
            self.write(self.base + off, fill)
        return self.base + off

    def put(self, array, align=256):
        a = np.ascontiguousarray(array)
        at = self.alloc(a.nbytes, align)
        self.write(at, a)
        return at

    def write(self, addr, array):
        a = np.ascontiguousarray(array).view(np.uint8).reshape(-1)
        off = addr - self.base
        self.t[off:off + a.size].copy_(torch.from_numpy(a.copy()))

    def get(self, addr, dtype, count):
        off = addr - self.base
        nbytes = np.dtype(dtype).itemsize * count
        torch.cuda.synchronize()
        return self.t[off:off + nbytes].cpu().numpy().view(dtype).copy()

    def reset(self):
        self.top = 0


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def first_difference(a, b):
    a = np.asarray(a, np.float32).reshape(-1)
    b = np.asarray(b, np.float32).reshape(-1)
    bad = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    if bad.size == 0:
        return "none"
    i = bad[0]
    return f"{bad.size} differ, first at {i}: {a[i]!r} vs {b[i]!r}"
