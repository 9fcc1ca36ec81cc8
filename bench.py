"""bench.py — the hot path's headline numbers on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-gemm] [--no-configs] [--configs]
                    [--mode phase|matmuls]
    python bench.py --profile gemm|gemm_wc|gemm_tol|gemv|gemv_m4   (one workload's launches alone, for rocprofv3's counters)
    python bench.py --profile blocks_decode|blocks_prompt [--block-type Q4_K]   (llama.cpp's blocks, the same way)
    python bench.py --calibrate     (kernels of known traffic, for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE)

A step is one decode token of the Llama-3-8B-shaped Q8 path: per layer the reference's
four phases (src/runtime/forward/attention.ts:173, ffn.ts:27-30): quantize_x of the input, then q / k / v
(4096, 1024, 1024 rows x 4096) in one phase, o (4096 x 4096), gate and up (2 x 14336 x 4096) in one phase, down
(4096 x 14336); 32 layers, then the classifier (128256 x 4096).  Every layer has its own weights (8.44 GB in all, far
past the 256 MB Infinity Cache), int8 uniform in [-127, 127] with |N(0, 0.02)| / 127 scales, activations N(0, 1):
synthetic, generated on the GPU from a seed.  The products are matmul_q8r's (relaxed form, quantize_x bias 64): a phase
is quantize_x of its input, then one hq_phase() call over the phase's jobs (the reference's ready() and phase()), the
corrections derived in the kernel (wc = NULL: the same integers as int8_sums' wc, and 1/9 fewer bytes).  Beside it:
the same step with the caller's wc (the reference's own call; its bytes counted), and through hq_matmuls() (the
reference's matmulsAlike: quantize_x into the jobs' a / b and the phase in one call; --mode matmuls makes it the
headline).

value: algorithmic bytes of a step (1.125 B a weight, the activations' bytes and scales, 4 B an output; jobs.ts:448-450)
over the step's time, with all inputs resident in HBM.  The step runs as a HIP graph of its launches (captured once).
roofline: the GEMV kernel alone: a graph of only a step's products launches, replayed between HIP events, gives its
average launch duration; traffic: the HBM bytes a launch moves, from rocprofv3's counters
(profiles/gemv_q8r_8b_decode_traffic.md).  Each kind of phase (q/k/v, o, gate/up, down, classifier) is also timed on
its own.
Also reported: config 3's decode at M = 4 (four tokens a step), the int8 prefill GEMM (config 3's M = 2048 over one
layer's matrices, corrections derived and the caller's) in TOPS against the dense int8 MFMA peak, the measured
ceilings (hq_ceiling_read past the caches, hq_ceiling_mfma on registers), configs 0, 1, 2 and 4, and
the CPU baseline: oracle/fast.c (the reference arithmetic, AVX2) on the host's cores, decode and prefill.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA
METRIC = "Q8 GEMV HBM GB/s (% peak) at 8B decode; int8 prefill GEMM TOPS (% MFMA)"

# Llama-3-8B
HIDDEN, FFN, LAYERS, VOCAB = 4096, 14336, 32, 128256
QKV_ROWS = (4096, 1024, 1024)


def load_package():
    sys.path.insert(0, ROOT)
    import __graft_entry__ as g
    return g.load_package()


class Matrix:
    """int8 weights (rows x n) and their scales on the GPU, with int8_sums' corrections on request."""

    def __init__(self, torch, gen, rows, n, wc=False):
        dev = "cuda:0"
        self.rows, self.n = rows, n
        self.w = torch.randint(-127, 128, (rows, n), dtype=torch.int8, device=dev, generator=gen)
        self.ws = (torch.randn(rows, n // 32, device=dev, generator=gen).abs_() * (0.02 / 127)).float()
        self.wc = torch.empty(rows, n // 32, dtype=torch.int32, device=dev) if wc else None

    def bytes(self):
        return self.rows * self.n * 1.125


class Activations:
    def __init__(self, torch, gen, n):
        dev = "cuda:0"
        self.n = n
        self.x = torch.randn(n, device=dev, generator=gen)
        self.xq = torch.empty(n, dtype=torch.uint8, device=dev)
        self.xs = torch.empty(n // 32, dtype=torch.float32, device=dev)

    def bytes(self):
        return self.n * 1.125  # int8 values and a float32 scale a group, read by the products


def build_decode(torch, jobs, lib):
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(3)
    acts = {n: Activations(torch, gen, n) for n in (HIDDEN, FFN)}
    layers = []
    for _ in range(LAYERS):
        layers.append({
            "qkv": [Matrix(torch, gen, r, HIDDEN, True) for r in QKV_ROWS],
            "o": [Matrix(torch, gen, HIDDEN, HIDDEN, True)],
            "gate_up": [Matrix(torch, gen, FFN, HIDDEN, True) for _ in range(2)],
            "down": [Matrix(torch, gen, HIDDEN, FFN, True)],
        })
    head = Matrix(torch, gen, VOCAB, HIDDEN, True)
    outs = {name: torch.empty(rows, dtype=torch.float32, device="cuda:0")
            for name, rows in (("q", 4096), ("k", 1024), ("v", 1024), ("o", HIDDEN), ("gate", FFN), ("up", FFN),
                               ("down", HIDDEN), ("logits", VOCAB))}
    for m in [m for layer in layers for ms in layer.values() for m in ms] + [head]:
        lib.hq_int8_sums_ex(m.wc.data_ptr(), m.w.data_ptr(), m.rows * m.n // 32, None)
    # the phases of one step, in decode order: (input activations, [(matrix, output)])
    phases = []
    for layer in layers:
        phases.append((acts[HIDDEN], list(zip(layer["qkv"], (outs["q"], outs["k"], outs["v"])))))
        phases.append((acts[HIDDEN], [(layer["o"][0], outs["o"])]))
        phases.append((acts[HIDDEN], list(zip(layer["gate_up"], (outs["gate"], outs["up"])))))
        phases.append((acts[FFN], [(layer["down"][0], outs["down"])]))
    phases.append((acts[HIDDEN], [(head, outs["logits"])]))
    return layers, head, phases


def phase_tables(jobs, phases, with_wc):
    """each phase as the reference's job table: (activations, table, jobs, algorithmic bytes (jobs.ts:448-450))"""
    tables = []
    for a, mats in phases:
        entries = [jobs.job("matmul_q8r", out.data_ptr(), a.xq.data_ptr(), a.xs.data_ptr(), m.w.data_ptr(),
                            m.ws.data_ptr(), m.wc.data_ptr() if with_wc else 0, m.n, rows=m.rows)
                   for m, out in mats]
        table = (ctypes.c_double * (16 * len(entries)))(*[float(v) for e in entries for v in e])
        # with the caller's wc the kernel also reads its int32 a group: 4 rows n / 32 bytes more
        bytes_ = sum(m.bytes() + (m.rows * m.n / 8 if with_wc else 0) + a.bytes() + 4 * m.rows for m, _ in mats)
        tables.append((a, table, len(entries), bytes_))
    return tables


def run_step(lib, tables, stream, matmuls, events=None):
    for i, (a, table, njobs, _) in enumerate(tables):
        if matmuls:  # engine.ts's matmulsAlike in one call: quantize_x into the jobs' a / b, then the phase
            if events is not None:
                events[i][0].record()
            lib.hq_matmuls(a.x.data_ptr(), 4 * a.n, table, njobs, 16, stream)
        else:  # quantize_x, then the phase
            lib.hq_quantize_x_ex(a.xq.data_ptr(), a.xs.data_ptr(), a.x.data_ptr(), a.n, 64, stream)
            if events is not None:
                events[i][0].record()
            lib.hq_phase(table, njobs, 16, stream)
        if events is not None:
            events[i][1].record()


PHASE_NAMES = ("qkv", "o", "gate_up", "down", "lm_head")


def measure_decode(torch, pkg, args, phases, matmuls, with_wc, by_phase=True):
    from pyodide_llm_amd import jobs
    lib = pkg.library()
    stream = torch.cuda.Stream()
    tables = phase_tables(jobs, phases, with_wc)
    step_bytes = sum(t[3] for t in tables)
    out = {"step_bytes": step_bytes}
    with torch.cuda.stream(stream):
        handle = stream.cuda_stream
        pkg.check(lib.hq_set_stream(handle))
        for _ in range(args.warmup):
            run_step(lib, tables, handle, matmuls)
        pkg.check(lib.hq_last_error())
        torch.cuda.synchronize()
        # the timed region: K steps as a HIP graph of one step's launches
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            run_step(lib, tables, handle, matmuls)
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            g.replay()
        torch.cuda.synchronize()
        graph_s = (time.perf_counter() - t0) / args.steps
        # the products alone: a graph of one step's products launches (no quantize_x; the activations are those the
        # last step left), replayed K times between HIP events on this stream.  Its launches run back to back, so
        # its time over its launches is the GEMV kernel's average duration (with the gaps between launches).
        def products(subset):
            gk = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gk, stream=stream):
                for a, table, njobs, _ in subset:
                    if matmuls:
                        lib.hq_matmuls(a.x.data_ptr(), 4 * a.n, table, njobs, 16, handle)
                    else:
                        lib.hq_phase(table, njobs, 16, handle)
            gk.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(args.steps):
                gk.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e-3 / args.steps

        gemv_s = products(tables)
        kinds = {}
        if by_phase:  # each kind of phase on its own (a graph of at least 32 launches)
            names = [PHASE_NAMES[i % 4] if i < 4 * LAYERS else "lm_head" for i in range(len(tables))]
            # the read ceiling on the same bytes: hq_ceiling_read over slices of one launch's bytes of the phase,
            # taken in turn from a 2 GiB buffer (several times the 256 MB Infinity Cache), a graph of 32 launches
            big = torch.empty(2 << 30, dtype=torch.uint8, device="cuda:0")
            sink = torch.zeros(256, dtype=torch.int32, device="cuda:0")
            for name in PHASE_NAMES:
                mine = [t for t, nm in zip(tables, names) if nm == name]
                mine = mine * -(-32 // len(mine))
                s = products(mine)
                size = int(sum(t[3] for t in mine) / len(mine)) // 16 * 16
                slices = big.numel() // size

                def reads(h, size=size, slices=slices):
                    for i in range(32):
                        lib.hq_ceiling_read(big.data_ptr() + (i % slices) * size, size, sink.data_ptr(), h)
                ceiling = _graph_time_median(torch, reads, max(5, args.steps)) / 32
                kinds[name] = {"us": round(1e6 * s / len(mine), 2),
                               "GBps": round(sum(t[3] for t in mine) / s / 1e9, 1),
                               "read_ceiling_us": round(1e6 * ceiling, 2),
                               "of_read_ceiling": round(s / len(mine) / ceiling, 3)}
            del big
        pkg.check(lib.hq_last_error())
        pkg.check(lib.hq_set_stream(None))
    out["ms_per_step"] = 1e3 * graph_s
    out["GBps"] = step_bytes / graph_s / 1e9
    out["gemv_avg_launch_us"] = 1e6 * gemv_s / len(tables)
    out["gemv_bytes_per_launch"] = step_bytes / len(tables)
    out["gemv_GBps"] = step_bytes / gemv_s / 1e9
    if kinds:
        out["phases"] = kinds
    return out


def build_decode_m4(torch, pkg, phases):
    """config 3's decode at M = 4: the same step for four tokens at once (each phase quantize_x of its input for the
    four tokens in one launch, then one hq_phase whose jobs take the four: every weight read once for four tokens).
    Returns step(stream) (the whole step), products(stream) (its hq_phase calls alone) and the step's algorithmic
    bytes: the weights, four tokens' activations, four outputs a row."""
    from pyodide_llm_amd import jobs
    lib = pkg.library()
    dev = "cuda:0"
    T = 4
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    acts = {}
    for a, _ in phases:
        if a.n not in acts:
            frame = (a.n + a.n // 8 + 15) // 16 * 16
            acts[a.n] = (torch.randn(T, a.n, device=dev, generator=gen),
                         torch.empty(T * frame, dtype=torch.uint8, device=dev), frame)
    outs = {}
    tables, step_bytes = [], 0.0
    for a, mats in phases:
        x, buf, frame = acts[a.n]
        entries = []
        for m, out in mats:
            o = outs.setdefault((m.rows, id(out)), torch.empty(T, m.rows, device=dev))
            entries.append(jobs.job("matmul_q8r", o.data_ptr(), buf.data_ptr(), buf.data_ptr() + a.n, m.w.data_ptr(),
                                    m.ws.data_ptr(), 0, m.n, rows=m.rows, count=T, os=4 * m.rows, as_=frame,
                                    bs=frame))
            step_bytes += m.bytes() + T * (a.bytes() + 4 * m.rows)
        tables.append((a.n, x, buf, frame, jobs.table(entries), len(entries)))

    def step(h):
        for n, x, buf, frame, table, njobs in tables:
            lib.hq_quantize_x_batch(buf.data_ptr(), buf.data_ptr() + n, x.data_ptr(), n, 64, T, frame, 4 * n, h)
            lib.hq_phase(table, njobs, 16, h)

    def products(h):
        for n, x, buf, frame, table, njobs in tables:
            lib.hq_phase(table, njobs, 16, h)
    return step, products, step_bytes, len(tables), outs


def measure_decode_m4(torch, pkg, args, phases):
    lib = pkg.library()
    step, products, step_bytes, launches, keep = build_decode_m4(torch, pkg, phases)
    reps = max(3, args.steps // 2)
    sec = _graph_time_median(torch, step, reps)
    gemv = _graph_time_median(torch, products, reps)
    pkg.check(lib.hq_last_error())
    return {"M": 4, "ms_per_step": round(1e3 * sec, 4), "GBps": round(step_bytes / sec / 1e9, 1),
            "tokens_per_s": round(4 / sec, 1), "step_bytes": step_bytes,
            "gemv_avg_launch_us": round(1e6 * gemv / launches, 3), "gemv_GBps": round(step_bytes / gemv / 1e9, 1)}


def _graph_time_median(torch, launch, reps, rounds=3):
    """the median of `rounds` measurements of _graph_time (one alone can be off by tens of per cent while the clocks
    settle)"""
    return sorted(_graph_time(torch, launch, reps) for _ in range(rounds))[rounds // 2]


def _graph_time(torch, launch, reps):
    """seconds a replay of a graph of launch()'s launches takes, over `reps` replays between HIP events"""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        launch(stream.cuda_stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            launch(stream.cuda_stream)
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / reps


def measure_configs(torch, pkg, args, extras):
    """The other configs' products on one GPU (BASELINE.json configs[0..2, 4], and config 4's shapes with binary
    weights, the packing the reference ranks next; with `extras` also llama.cpp's blocks and the classifier's outlier
    channels): GB/s of algorithmic bytes for the token products (M = 1; copies of the weights past the Infinity Cache
    where the shapes allow), TOPS for the prompts.  Products only (the activations prepared once), graphs of their
    launches timed with HIP events."""
    from pyodide_llm_amd import jobs
    lib = pkg.library()
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(11)
    dev = "cuda:0"
    reps = max(3, args.steps // 2)
    out = {}

    def acts(n, kind, count=1):
        x = torch.randn(count, n, device=dev, generator=gen)
        area = (8 if kind in ("ternary", "binary") else 4) * (n // 32)
        frame = (n + area + 15) // 16 * 16
        buf = torch.empty(count * frame, dtype=torch.uint8, device=dev)
        bias = 64 if kind in ("int8", "int6") else 0
        pkg.check(lib.hq_quantize_x_batch(buf.data_ptr(), buf.data_ptr() + n, x.data_ptr(), n, bias, count, frame,
                                          4 * n, None))
        if kind in ("ternary", "binary"):
            pkg.check(lib.hq_interleave_batch(buf.data_ptr(), buf.data_ptr() + n, n, count, frame, None))
        return buf, frame

    def weights(kind, rows, n):
        if kind == "int8":
            w = torch.randint(-127, 128, (rows, n), dtype=torch.int8, device=dev, generator=gen)
            ws = (torch.randn(rows, n // 32, device=dev, generator=gen).abs_() * (0.02 / 127)).float()
        elif kind == "int6":  # random bytes are valid packed int6 groups
            w = torch.randint(0, 256, (rows, n // 32 * 24), dtype=torch.uint8, device=dev, generator=gen)
            ws = (torch.randn(rows, n // 32, device=dev, generator=gen).abs_() * (0.02 / 124)).float()
        else:  # ternary: codes 0..2 four to a byte; binary: random bytes (a bit a sign); a float16 scale a row
            if kind == "ternary":
                codes = torch.randint(0, 3, (rows, n // 4, 4), dtype=torch.uint8, device=dev, generator=gen)
                w = (codes[..., 0] | (codes[..., 1] << 2) | (codes[..., 2] << 4) | (codes[..., 3] << 6)).contiguous()
            else:
                w = torch.randint(0, 256, (rows, n // 8), dtype=torch.uint8, device=dev, generator=gen)
            row = (torch.randn(rows, 1, device=dev, generator=gen).abs_() * 0.02 + 1e-3).half()
            ws = row.expand(rows, n // 128).contiguous()
        return w, ws

    per_weight = {"int8": 1.125, "int6": 0.875, "ternary": 0.265625, "binary": 0.140625}
    kind_name = {"int8": "matmul_q8r", "int6": "matmul_q6r", "ternary": "matmul_t2r", "binary": "matmul_b1r"}

    def decode(label, kind, phase_shapes, copies):
        """phase_shapes: [[(rows, n), ...] a phase]; `copies` sets of distinct weights, every phase of each"""
        a = {n: acts(n, kind) for ph in phase_shapes for _, n in ph}
        tables, total = [], 0.0
        keep = []
        for _ in range(copies):
            for ph in phase_shapes:
                entries = []
                for rows, n in ph:
                    w, ws = weights(kind, rows, n)
                    o = torch.empty(rows, device=dev)
                    keep += [w, ws, o]
                    buf, frame = a[n]
                    # wc 0: the corrections derived in the kernel (int8, int6); ternary jobs have none
                    entries.append(jobs.job(kind_name[kind], o.data_ptr(), buf.data_ptr(), buf.data_ptr() + n,
                                            w.data_ptr(), ws.data_ptr(), 0, n, rows=rows))
                    total += rows * n * per_weight[kind] + n * (1.25 if kind in ("ternary", "binary") else 1.125) + 4 * rows
                tables.append((jobs.table(entries), len(entries)))

        def launch(h):
            for t, nj in tables:
                lib.hq_phase(t, nj, 16, h)
        sec = _graph_time_median(torch, launch, reps)
        pkg.check(lib.hq_last_error())
        out[label] = {"GBps": round(total / sec / 1e9, 1), "us_per_launch": round(1e6 * sec / len(tables), 2),
                      "launches": len(tables), "bytes": total}

    def prefill(label, kind, shapes, count, tol=False, caller_wc=True):
        """caller_wc (int8): the reference's own call, the corrections int8_sums made (tensors.ts:126-132); else
        derived in the tile.  tol: hq_matmul_q8r_tile_tol_ex, whose launches of fewer tiles than two blocks a compute
        unit take the bit-exact tile with derived corrections (hq_tol_min_tiles' default): which did is reported"""
        ops, calls, keep = 0.0, [], []
        cus = torch.cuda.get_device_properties(0).multi_processor_count
        tol_tiles = [((r + 127) // 128) * ((count + 127) // 128) for r, _ in shapes]
        if tol:  # the tolerance form's workspace, one for the calls, which follow each other on the stream
            need = max(lib.hq_tol_work_bytes(n, count) for _, n in shapes)
            work = torch.empty(need + 256, dtype=torch.uint8, device=dev)
            wptr = (work.data_ptr() + 255) // 256 * 256
            keep.append(work)
        for rows, n in shapes:
            w, ws = weights(kind, rows, n)
            buf, frame = acts(n, kind, count)
            o = torch.empty(count, rows, device=dev)
            keep += [w, ws, buf, o]
            ops += 2.0 * count * rows * n
            if tol:
                calls.append(lambda h, w=w, ws=ws, buf=buf, frame=frame, o=o, rows=rows, n=n:
                             lib.hq_matmul_q8r_tile_tol_ex(o.data_ptr(), buf.data_ptr(), buf.data_ptr() + n,
                                                           w.data_ptr(), ws.data_ptr(), n, 0, rows, count, 4 * rows,
                                                           frame, wptr, need, h))
            elif kind == "int8":
                wc = torch.empty(rows, n // 32, dtype=torch.int32, device=dev)
                pkg.check(lib.hq_int8_sums_ex(wc.data_ptr(), w.data_ptr(), rows * n // 32, None))
                keep.append(wc)
                if not caller_wc:
                    wc = None
                calls.append(lambda h, w=w, ws=ws, wc=wc, buf=buf, frame=frame, o=o, rows=rows, n=n:
                             lib.hq_matmul_q8r_tile_ex(o.data_ptr(), buf.data_ptr(), buf.data_ptr() + n, w.data_ptr(),
                                                       ws.data_ptr(), wc.data_ptr() if wc is not None else None, n, 0,
                                                       rows, count, 4 * rows, frame, h))
            elif kind == "ternary":
                calls.append(lambda h, w=w, ws=ws, buf=buf, frame=frame, o=o, rows=rows, n=n:
                             lib.hq_matmul_t2r_tile_ex(o.data_ptr(), buf.data_ptr(), buf.data_ptr() + n, w.data_ptr(),
                                                       ws.data_ptr(), n, 0, rows, count, 4 * rows, frame, 3, h))
            elif kind == "binary":
                calls.append(lambda h, w=w, ws=ws, buf=buf, frame=frame, o=o, rows=rows, n=n:
                             lib.hq_matmul_b1r_tile_ex(o.data_ptr(), buf.data_ptr(), buf.data_ptr() + n, w.data_ptr(),
                                                       ws.data_ptr(), n, 0, rows, count, 4 * rows, frame, 2, h))
            else:
                t = jobs.table([jobs.job("matmul_q6r", o.data_ptr(), buf.data_ptr(), buf.data_ptr() + n, w.data_ptr(),
                                         ws.data_ptr(), 0, n, rows=rows, count=count, os=4 * rows, as_=frame,
                                         bs=frame)])
                keep.append(t)
                calls.append(lambda h, t=t: lib.hq_phase(t, 1, 16, h))

        def launch(h):
            for c in calls:
                c(h)
        sec = _graph_time_median(torch, launch, reps)
        pkg.check(lib.hq_last_error())
        out[label] = {"TOPS": round(ops / sec / 1e12, 1), "frac": round(ops / sec / 1e12 / INT8_PEAK_TOPS, 4),
                      "ms": round(1e3 * sec, 3)}
        if tol:
            out[label]["launches_on_the_tolerance_tile"] = sum(t >= 2 * cus for t in tol_tiles)
            out[label]["launches"] = len(shapes)

    decode("c0 stories15M q8r M=1 (weights in cache: 221 KB x 64)", "int8", [[(768, 288)]], 64)
    decode("c1 LFM2-350M q8r M=1, 16 layers + lm-head", "int8",
           [[(1536, 1024)], [(1024, 1024)], [(9216, 1024)], [(1024, 4608)]] * 16 + [[(65536, 1024)]], 1)
    c2 = [(3072, 2048), (2048, 2048), (8192, 2048), (8192, 2048), (2048, 8192)]
    prefill("c2 Llama-3.2-1B prefill M=512, one layer (the caller's wc)", "int8", c2, 512)
    prefill("c2 Llama-3.2-1B prefill M=512, one layer (corrections derived)", "int8", c2, 512, caller_wc=False)
    prefill("c2 Llama-3.2-1B prefill M=512, one layer, tolerance entry point", "int8", c2, 512, tol=True)
    for kind in ("ternary", "int6", "binary"):
        copies = {"ternary": 8, "int6": 3, "binary": 12}[kind]
        tag = "c4 27B" if kind != "binary" else "27B shapes"
        decode(f"{tag} {kind} M=1, gate+up x {copies}", kind, [[(17408, 5120), (17408, 5120)]], copies)
        decode(f"{tag} {kind} M=1, down x {copies}", kind, [[(5120, 17408)]], copies)
        prefill(f"{tag} {kind} prefill M=256", kind, [(17408, 5120), (17408, 5120), (5120, 17408)], 256)
    if extras:
        out.update(measure_blocks(torch, pkg, args, gen))
        out.update(measure_outliers(torch, pkg, args, gen))
    return out


def measure_outliers(torch, pkg, args, gen):
    """The classifier's outlier channels (engine.ts:459-466): add_columns alone (8 columns of GPT-2's 50257 and
    Llama-3's 128256 words: GB/s of its 4 vocab (count + 2) bytes), and Llama-3-8B's classifier of one token
    ([128256, 4096] int8) with the 8 channels taken apart, the product and add_columns, against the product alone."""
    import ctypes
    from pyodide_llm_amd import jobs
    lib = pkg.library()
    dev = "cuda:0"
    reps = max(3, args.steps // 2)
    out = {}
    count = 8
    channels = (ctypes.c_int32 * count)(*[1, 50, 300, 777, 1024, 2000, 3000, 4095])
    for vocab in (50257, 128256):
        y = torch.randn(vocab, device=dev, generator=gen)
        rows = torch.randn(count, vocab, device=dev, generator=gen)
        a = torch.randn(count, device=dev, generator=gen)
        def launches(h, y=y, rows=rows, a=a, vocab=vocab):  # 50 back to back: a graph's own cost is not the kernel's
            for _ in range(50):
                lib.hq_add_columns_ex(y.data_ptr(), rows.data_ptr(), a.data_ptr(), count, vocab, h)
        sec = _graph_time(torch, launches, reps) / 50
        pkg.check(lib.hq_last_error())
        out[f"add_columns {count} x {vocab}"] = {"GBps": round(4 * vocab * (count + 2) / sec / 1e9, 1),
                                                 "us": round(1e6 * sec, 2)}
    vocab, dim = 128256, 4096
    w = torch.randint(-127, 128, (vocab, dim), dtype=torch.int8, device=dev, generator=gen)
    ws = (torch.rand(vocab, dim // 32, device=dev, generator=gen) * 0.001).float()
    x = torch.randn(dim, device=dev, generator=gen)
    logits = torch.empty(vocab, device=dev)
    xq = torch.empty(2 * dim, dtype=torch.uint8, device=dev)
    columns = torch.empty(count, vocab, device=dev)
    picked = torch.empty(count, device=dev)
    pkg.check(lib.hq_outlier_columns_ex(columns.data_ptr(), w.data_ptr(), ws.data_ptr(), 0, channels, count, vocab,
                                        dim, None))
    table = jobs.table([jobs.job("matmul_q8r", logits.data_ptr(), xq.data_ptr(), xq.data_ptr() + dim, w.data_ptr(),
                                 ws.data_ptr(), 0, dim, rows=vocab)])

    def product(h):
        lib.hq_matmuls(x.data_ptr(), 4 * dim, table, 1, 16, h)

    def classify(h):
        lib.hq_take_channels_ex(picked.data_ptr(), x.data_ptr(), channels, count, h)
        product(h)
        lib.hq_add_columns_ex(logits.data_ptr(), columns.data_ptr(), picked.data_ptr(), count, vocab, h)
    alone = _graph_time(torch, product, reps)
    apart = _graph_time(torch, classify, reps)
    pkg.check(lib.hq_last_error())
    out["8B classifier, 8 outlier channels apart"] = {"us": round(1e6 * apart, 2), "us_product_alone":
                                                      round(1e6 * alone, 2)}
    return out


# where each block type keeps its float16 scales (kernels/blocks/types.ts:60-79): set to 2^-7 in the synthetic
# blocks so that every product is finite; IQ1_M's is spread over the top nibbles of the words at 48..55
BLOCK_SCALES = {10: (80, 82), 12: (0, 2), 16: (0,), 17: (0,), 18: (0,), 19: (0,), 21: (0,), 22: (0,), 23: (0,)}


class BlocksWorkload:
    """llama.cpp's blocks (job kinds 10-12) at Llama-3-8B's MLP shapes (gate, up [14336, 4096], down [4096, 14336]):
    random blocks (random bytes, sane scales), random codebooks, activations quantized with their sums."""
    SHAPES = [(14336, 4096), (14336, 4096), (4096, 14336)]

    def __init__(self, torch, pkg, gen):
        self.torch, self.pkg, self.gen = torch, pkg, gen
        self.lib = pkg.library()
        self.dev = "cuda:0"
        self.tab = torch.empty(34992, dtype=torch.uint8, device=self.dev)
        books = torch.randint(0, 256, (33808,), dtype=torch.uint8, device=self.dev, generator=gen)
        pkg.check(self.lib.hq_sb_tables_ex(self.tab.data_ptr(), books.data_ptr(), None))

    def acts(self, n, count=1):
        x = self.torch.randn(count, n, device=self.dev, generator=self.gen)
        frame = (n + n // 2 + 15) // 16 * 16
        buf = self.torch.empty(count * frame, dtype=self.torch.uint8, device=self.dev)
        self.pkg.check(self.lib.hq_quantize_x_batch(buf.data_ptr(), buf.data_ptr() + n, x.data_ptr(), n, 0, count,
                                                    frame, 4 * n, None))
        self.pkg.check(self.lib.hq_sums_x_batch(buf.data_ptr() + n, buf.data_ptr(), n, count, frame, None))
        return buf, frame

    def weights(self, t, size, rows, n):
        w = self.torch.randint(0, 256, (rows * (n // 256), size), dtype=self.torch.uint8, device=self.dev,
                               generator=self.gen)
        for at in BLOCK_SCALES.get(t, ()):
            w[:, at], w[:, at + 1] = 0x00, 0x20
        if t == 29:  # 0x2000: the nibbles 0, 0, 0, 2 at the tops of the four words
            for k, nib in enumerate((0, 0, 0, 2)):
                w[:, 49 + 2 * k] = (w[:, 49 + 2 * k] & 0x0F) | (nib << 4)
        return w

    @staticmethod
    def act_bytes(t, n):
        """per token: xq, the scales, and the sums of 16 (the K types) or of 8 (IQ1)"""
        return n + n // 8 + (n // 8 if t in (10, 12) else n // 4 if t in (19, 29) else 0)

    def decode(self, name):
        """the token product (M = 1) of `copies` copies of one layer's MLP (together past the Infinity Cache), gate
        and up in one phase, down in the next (their launches as the forward pass makes them).  Returns launch(h),
        the launches a call, the copies and the algorithmic bytes a call (the blocks, the activations and sums the
        type reads, the outputs)."""
        from pyodide_llm_amd import jobs
        t, size = jobs.BLOCK_TYPES[name]
        per_layer = sum(rows * (n // 256) * size for rows, n in self.SHAPES)
        copies = max(2, -(-1_200_000_000 // per_layer))
        a = {n: self.acts(n) for _, n in self.SHAPES}
        tables, total, keep = [], 0.0, []
        for _ in range(copies):
            entries = []
            for rows, n in self.SHAPES:
                w = self.weights(t, size, rows, n)
                o = self.torch.empty(rows, device=self.dev)
                keep += [w, o]
                buf, _ = a[n]
                entries.append(jobs.job("matmul_sbr", o.data_ptr(), buf.data_ptr(), buf.data_ptr() + n, w.data_ptr(),
                                        self.tab.data_ptr(), t, n, rows=rows))
                total += rows * (n // 256) * size + self.act_bytes(t, n) + 4 * rows
            tables.append((jobs.table(entries[:2]), 2))
            tables.append((jobs.table(entries[2:]), 1))
        lib = self.lib

        def launch(h, keep=keep, a=a):
            for tb, nj in tables:
                lib.hq_phase(tb, nj, 16, h)
        return launch, len(tables), copies, total

    def prompt(self, name, count):
        """a prompt of `count` tokens through one layer's MLP (one hq_phase of three jobs: the matrix-core tile).
        Returns launch(h) and the operations a call."""
        from pyodide_llm_amd import jobs
        t, size = jobs.BLOCK_TYPES[name]
        entries, keep = [], []
        for rows, n in self.SHAPES:
            w = self.weights(t, size, rows, n)
            buf, frame = self.acts(n, count)
            o = self.torch.empty(count, rows, device=self.dev)
            keep += [w, buf, o]
            entries.append(jobs.job("matmul_sbr", o.data_ptr(), buf.data_ptr(), buf.data_ptr() + n, w.data_ptr(),
                                    self.tab.data_ptr(), t, n, rows=rows, count=count, os=4 * rows, as_=frame,
                                    bs=frame))
        tb = jobs.table(entries)
        lib = self.lib

        def launch(h, keep=keep):
            lib.hq_phase(tb, len(entries), 16, h)
        return launch, sum(2.0 * count * rows * n for rows, n in self.SHAPES)


def measure_blocks(torch, pkg, args, gen, names=None, prompts=None):
    """llama.cpp's blocks at Llama-3-8B's MLP shapes: the token product (M = 1) in GB/s of algorithmic bytes and
    prompts of 64 and 512 tokens in TOPS, every block type (or `names`, prompts of `prompts` tokens)."""
    from pyodide_llm_amd import jobs
    lib = pkg.library()
    reps = max(3, args.steps // 2)
    out = {}
    W = BlocksWorkload(torch, pkg, gen)
    for name in names or jobs.BLOCK_TYPES:
        launch, _, copies, total = W.decode(name)
        sec = _graph_time(torch, launch, reps)
        pkg.check(lib.hq_last_error())
        out[f"8B MLP {name} M=1 x {copies}"] = {"GBps": round(total / sec / 1e9, 1),
                                                  "us_per_layer": round(1e6 * sec / copies, 2), "bytes": total}
        del launch
        for count in prompts or getattr(args, "block_prompts", (64, 512)):
            launch, ops = W.prompt(name, count)
            sec = _graph_time(torch, launch, reps)
            pkg.check(lib.hq_last_error())
            out[f"8B MLP {name} prompt M={count}"] = {"TOPS": round(ops / sec / 1e12, 2), "ms": round(1e3 * sec, 3)}
            del launch
            torch.cuda.empty_cache()
    return out


def gemm_workload(torch, pkg):
    """config 3's prefill: M = 2048 tokens through one layer's matrices (q, k, v, o, gate, up, down), the activations
    quantized once.  Returns run(with_wc) (the 7 products on the null stream: corrections derived in the kernel,
    wc = NULL, as the headline GEMV runs, or the caller's, int8_sums' as the reference's loader makes them,
    tensors.ts:126-134; the same numbers either way), the launches of a run, and its int8 operations."""
    lib = pkg.library()
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(5)
    M = 2048
    shapes = [(4096, HIDDEN), (1024, HIDDEN), (1024, HIDDEN), (HIDDEN, HIDDEN), (FFN, HIDDEN), (FFN, HIDDEN),
              (HIDDEN, FFN)]
    mats = [Matrix(torch, gen, r, n, wc=True) for r, n in shapes]
    for m in mats:
        pkg.check(lib.hq_int8_sums_ex(m.wc.data_ptr(), m.w.data_ptr(), m.rows * m.n // 32, None))
    acts = {}
    for n in (HIDDEN, FFN):
        x = torch.randn(M, n, device="cuda:0", generator=gen)
        frame = n + 4 * (n // 32)
        buf = torch.empty(M * frame, dtype=torch.uint8, device="cuda:0")
        pkg.check(lib.hq_quantize_x_batch(buf.data_ptr(), buf.data_ptr() + n, x.data_ptr(), n, 64, M, frame, 4 * n, None))
        acts[n] = (buf, frame)
    outs = [torch.empty(M, r, dtype=torch.float32, device="cuda:0") for r, _ in shapes]
    # the tolerance form's workspace (the activations widened to float16, the scales regrouped), one for the layer's
    # calls, which follow each other on the null stream
    need = max(lib.hq_tol_work_bytes(n, M) for n in (HIDDEN, FFN))
    work = torch.empty(need + 256, dtype=torch.uint8, device="cuda:0")
    wptr = (work.data_ptr() + 255) // 256 * 256

    def run(with_wc, tol=False):
        for m, o in zip(mats, outs):
            buf, frame = acts[m.n]
            if tol:
                lib.hq_matmul_q8r_tile_tol_ex(o.data_ptr(), buf.data_ptr(), buf.data_ptr() + m.n, m.w.data_ptr(),
                                              m.ws.data_ptr(), m.n, 0, m.rows, M, 4 * m.rows, frame, wptr, need, None)
            else:
                lib.hq_matmul_q8r_tile_ex(o.data_ptr(), buf.data_ptr(), buf.data_ptr() + m.n, m.w.data_ptr(),
                                          m.ws.data_ptr(), m.wc.data_ptr() if with_wc else None, m.n, 0, m.rows, M,
                                          4 * m.rows, frame, None)
    run.keep = (mats, acts, outs, work)
    return run, len(shapes), sum(2.0 * M * r * n for r, n in shapes)


def measure_gemm(torch, pkg, args):
    """the prefill GEMM in TOPS: gemm_workload's layer, both forms taking turns (5 rounds of `steps` layers each, the
    median round's rate: one round alone varies by several per cent)"""
    lib = pkg.library()
    run, _, ops = gemm_workload(torch, pkg)
    forms = {"exact": lambda: run(False), "exact_with_wc": lambda: run(True), "tolerance": lambda: run(False, True)}
    times = {k: [] for k in forms}
    for f in forms.values():
        f()
    pkg.check(lib.hq_last_error())
    torch.cuda.synchronize()
    # the tolerance form's outputs against the bit-exact tile's (the reference's numbers), matrix by matrix
    mats, _, outs, _ = run.keep
    run(False)
    exact = [o.clone() for o in outs]
    run(False, True)
    torch.cuda.synchronize()
    worst = max(float((o - e).abs().max() / e.abs().max()) for o, e in zip(outs, exact))
    reps = max(5, args.steps)
    for _ in range(5):
        for name, f in forms.items():
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                f()
            e1.record()
            torch.cuda.synchronize()
            times[name].append(e0.elapsed_time(e1) * 1e-3 / reps)
    pkg.check(lib.hq_last_error())
    out = {"M": 2048}
    for name in forms:
        s = sorted(times[name])[2]
        r = {"tops": round(ops / s / 1e12, 1), "frac": round(ops / s / 1e12 / INT8_PEAK_TOPS, 4),
             "ms_per_layer": round(s * 1e3, 4), "best_tops": round(ops / min(times[name]) / 1e12, 1)}
        if name == "exact":
            out.update(r)
        elif name == "exact_with_wc":
            out["with_wc"] = r
        else:
            r.update({"kernel": "gemm_tol (float16-operand MFMA, one fused multiply-add a group; its activation "
                                "widening included)",
                      "max_err_over_max_y": worst, "bound": 1e-5})
            out["tolerance"] = r
    return out


def cpu_description():
    """the host's CPU model, its logical CPUs and the CPUs this process may run on"""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count() or 1, len(os.sched_getaffinity(0))


# the reference's own CPU figures (one thread, WebAssembly relaxed SIMD on an Ampere A1 Neoverse-N1,
# docs/notes/t158-cpu-audit-2026-09-27.md:5): :36 matmul_q8r out of the caches, :39 the prompt's blocks
REFERENCE_CPU = {"matmul_q8r_GBps_per_thread": "11.4-11.5 (t158:36, 51-75 MB matrices)",
                 "matmul_q8r_tile_GMACps_per_thread": "15.0-15.8 (t158:39, 16-token blocks)"}


def cpu_baseline(args, gemv_seconds=8.0, tile_seconds=6.0):
    """The CPU baseline: oracle/fast.c, the reference's relaxed int8 arithmetic vectorised for x86-64 (AVX2; every
    output the oracle's, tests/test_oracle.py), on the host threads one GPU's share allows (at most 16), rows cut as
    the reference's phase() cuts them (threads.ts:45, 109-110).
      GEMV: matmul_q8r with the caller's wc (as the reference's loader passes it) over two Llama-3-8B layers' 7
        matrices (490 MB, read in turn: past a socket's last-level cache as tests/tile-bench.ts:15-17 asks), pass
        after pass for about gemv_seconds: GB/s of the bytes a pass reads (1.25 B a weight, activations, outputs).
      prefill: matmul_q8r_tile of config 3's M = 2048 tokens over one layer's 7 matrices (4 rows x 4 tokens a
        step), pass after pass for about tile_seconds: TOPS = 2 M N K / time."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    model, nproc, allowed = cpu_description()
    threads = min(16, allowed)
    rng = np.random.default_rng(9)
    shapes = [(4096, HIDDEN), (1024, HIDDEN), (1024, HIDDEN), (HIDDEN, HIDDEN), (FFN, HIDDEN), (FFN, HIDDEN),
              (HIDDEN, FFN)]
    mats = []
    for _ in range(2):
        for rows, n in shapes:
            w = rng.integers(-127, 128, rows * n, dtype=np.int8)
            ws = (np.abs(rng.standard_normal(rows * n // 32)) * 0.02 / 127).astype(np.float32)
            mats.append((rows, n, w, ws, oracle.int8_sums(w)))
    acts = {n: oracle.quantize_x(rng.standard_normal(n).astype(np.float32), 64) for n in (HIDDEN, FFN)}
    gemv_s, gemv_bytes, passes = 0.0, 0.0, 0
    while gemv_s < gemv_seconds:
        for rows, n, w, ws, wc in mats:
            xq, xs = acts[n]
            gemv_s += oracle.time_fast_q8r(xq, xs, w, ws, wc, n, rows, threads)
            gemv_bytes += rows * n * 1.25 + n * 1.125 + 4 * rows
        passes += 1
    M = 2048
    frames = {}
    for n in (HIDDEN, FFN):
        frame = n + n // 8
        buf = np.zeros((M, frame), np.uint8)
        x = rng.standard_normal((M, n)).astype(np.float32)
        for t in range(M):
            q, sc = oracle.quantize_x(x[t], 64)
            buf[t, :n], buf[t, n:] = q, sc.view(np.uint8)
        frames[n] = (buf, frame)
    tile_s, tile_ops, tile_passes = 0.0, 0.0, 0
    while tile_s < tile_seconds:
        for rows, n, w, ws, wc in mats[:7]:
            buf, frame = frames[n]
            tile_s += oracle.time_fast_q8r(buf, buf[:, n:], w, ws, wc, n, rows, threads, count=M, frame=frame)
            tile_ops += 2.0 * M * rows * n
        tile_passes += 1
    gbps = gemv_bytes / gemv_s / 1e9
    return {"value": round(gbps, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"oracle/fast.c matmul_q8r (AVX2, the oracle's numbers) with wc over two Llama-3-8B layers' 7 "
                      f"matrices at M=1 (490 MB read in turn), {passes} passes in {gemv_s:.1f} s on {threads} "
                      f"threads",
            "per_thread_GBps": round(gbps / threads, 2),
            "prefill": {"TOPS": round(tile_ops / tile_s / 1e12, 3), "M": M,
                        "per_thread_GMACps": round(tile_ops / 2 / tile_s / 1e9 / threads, 1),
                        "sample": f"matmul_q8r_tile over one layer's 7 matrices, {tile_passes} passes in "
                                  f"{tile_s:.1f} s"},
            "cpu_model": model, "nproc": nproc, "cpus_allowed": allowed, "reference": REFERENCE_CPU}


def measure_ceilings(torch, pkg):
    """The measured ceilings beside the nominal peaks: hq_ceiling_read over 512 MB buffers taken in turn (2 GB in
    all, past the 256 MB Infinity Cache; a graph of 16 launches), hq_ceiling_mfma (registers only, 8 blocks a CU),
    and hq_ceiling_epilogue's two forms (the prompt tiles' register work, 2 blocks a CU as the tiles run)."""
    lib = pkg.library()
    sink = torch.zeros(256, dtype=torch.int32, device="cuda:0")
    size = 512 << 20
    bufs = [torch.ones(size, dtype=torch.uint8, device="cuda:0") for _ in range(4)]

    def reads(h):
        for i in range(16):
            pkg.check(lib.hq_ceiling_read(bufs[i % 4].data_ptr(), size, sink.data_ptr(), h))
    read_s = _graph_time(torch, reads, 3) / 16
    del bufs
    torch.cuda.empty_cache()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks, iters = 8 * cus, 2000

    def mfmas(h):
        pkg.check(lib.hq_ceiling_mfma(blocks, iters, sink.data_ptr(), h))
    mfma_s = _graph_time(torch, mfmas, 3)
    ops = blocks * 4 * iters * 8 * 32768 * 2
    # the prompt tiles' epilogues on registers, two waves a SIMD (2 blocks a CU)
    eblocks, eiters = 2 * cus, 4000
    epilogue = {}
    for form, name in ((0, "epilogue_exact_TOPS"), (1, "epilogue_tolerance_TOPS")):
        def work(h, form=form):
            pkg.check(lib.hq_ceiling_epilogue(form, eblocks, eiters, sink.data_ptr(), h))
        es = _graph_time_median(torch, work, 3)
        epilogue[name] = round(eblocks * 4 * eiters * 262144 / es / 1e12, 1)
    return {"read_GBps": round(size / read_s / 1e9, 1), "read_bytes": size,
            "mfma_int8_TOPS": round(ops / mfma_s / 1e12, 1), **epilogue}


def calibrate():
    """Kernels of known traffic for the counters' scale: a device-to-device copy of 1 GiB (reads and writes 1 GiB)
    and hq_ceiling_read over the same GiB (reads it), three times each."""
    import torch
    pkg = load_package()
    lib = pkg.library()
    size = 1 << 30
    a = torch.empty(size, dtype=torch.uint8, device="cuda:0").fill_(1)
    b = torch.empty_like(a)
    sink = torch.zeros(256, dtype=torch.int32, device="cuda:0")
    for _ in range(3):
        b.copy_(a)
        pkg.check(lib.hq_ceiling_read(a.data_ptr(), size, sink.data_ptr(), None))
    torch.cuda.synchronize()
    print(json.dumps({"calibrate": {"copy_bytes_read": size, "copy_bytes_written": size, "read_kernel_bytes": size}}))


def traffic_per_launch():
    """HBM bytes a launch of the headline GEMV kernel moves, as rocprofv3's FETCH_SIZE and WRITE_SIZE counted them
    (scaled by the same counters over a copy of known size), from the summary in profiles/; None without one."""
    path = os.path.join(ROOT, "profiles", "gemv_q8r_8b_decode_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def profile(torch, pkg, args):
    """--profile WHAT: WHAT's launches alone, issued directly (no graph) `steps` times after `warmup` untimed ones,
    for rocprofv3's counters (a counter pass serialises the dispatches):
      gemm     config 3's prefill, M = 2048 through one layer's 7 matrices, corrections derived (gemm_relaxed)
      gemm_wc  the same with the caller's corrections (int8_sums')
      gemm_tol the same in the tolerance form (tol_prepare_x / _s, then gemm_tol)
      gemv     one decode step's products at M = 1 (129 hq_phase launches of gemv_relaxed<8,1,...>)
      gemv_m4  the same at M = 4 (gemv_relaxed<8,4,...>)
      blocks_decode  --block-type's token product at M = 1 through copies of Llama-3-8B's MLP (sb_gemv)
      blocks_prompt  --block-type's prompt of 512 tokens through one layer's MLP (the matrix-core tile)
    Prints one JSON line naming what ran."""
    from pyodide_llm_amd import jobs
    lib = pkg.library()
    if args.profile in ("gemm", "gemm_wc", "gemm_tol"):
        run, launches, _ = gemm_workload(torch, pkg)
        for _ in range(args.warmup + args.steps):
            run(args.profile == "gemm_wc", args.profile == "gemm_tol")
    elif args.profile in ("blocks_decode", "blocks_prompt"):
        gen = torch.Generator(device="cuda:0")
        gen.manual_seed(12)
        W = BlocksWorkload(torch, pkg, gen)
        if args.profile == "blocks_decode":
            launch, launches, _, _ = W.decode(args.block_type)
        else:
            launch, _ = W.prompt(args.block_type, 512)
            launches = 1
        torch.cuda.synchronize()
        for _ in range(args.warmup + args.steps):
            launch(None)
    else:
        layers, head, phases = build_decode(torch, jobs, lib)
        if args.profile == "gemv":
            tables = phase_tables(jobs, phases, False)
            for a, _ in phases:  # the activations the products read
                pkg.check(lib.hq_quantize_x_ex(a.xq.data_ptr(), a.xs.data_ptr(), a.x.data_ptr(), a.n, 64, None))

            def products(h):
                for a, table, njobs, _ in tables:
                    lib.hq_phase(table, njobs, 16, h)
            launches = len(tables)
        else:
            step, products, _, launches, keep = build_decode_m4(torch, pkg, phases)
            step(None)
        for _ in range(args.warmup + args.steps):
            products(None)
    torch.cuda.synchronize()
    pkg.check(lib.hq_last_error())
    line = {"profile": args.profile, "launches_per_step": launches, "steps": args.warmup + args.steps}
    if args.profile.startswith("blocks"):
        line["block_type"] = args.block_type
    print(json.dumps(line))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip configs 0, 1, 2 and 4")
    ap.add_argument("--mode", choices=("phase", "matmuls"), default="phase",
                    help="the headline's phases: quantize_x then hq_phase (the reference's ready() + phase()), or "
                         "hq_matmuls (the same in one call, the reference's matmulsAlike)")
    ap.add_argument("--configs", action="store_true",
                    help="also measure llama.cpp's blocks (all ten types) and the outlier channels")
    ap.add_argument("--profile", choices=("gemm", "gemm_wc", "gemm_tol", "gemv", "gemv_m4", "blocks_decode",
                                          "blocks_prompt"),
                    help="only run one workload's launches, for rocprofv3's counters")
    ap.add_argument("--block-type", default="Q4_K",
                    help="the llama.cpp block type of --profile blocks_decode / blocks_prompt (a BLOCK_TYPES name)")
    ap.add_argument("--calibrate", action="store_true",
                    help="only run kernels of known traffic (for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.calibrate:
        calibrate()
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: the path is built for one MI355X (rows would shard across GPUs with an "
              "all-gather of the outputs, which this build does not run); use --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    pkg = load_package()
    torch.cuda.set_device(0)
    pkg.check(pkg.library().hq_init())
    if args.profile:
        profile(torch, pkg, args)
        return
    from pyodide_llm_amd import jobs
    layers, head, phases = build_decode(torch, jobs, pkg.library())
    separate = measure_decode(torch, pkg, args, phases, matmuls=False, with_wc=False)
    separate_wc = measure_decode(torch, pkg, args, phases, matmuls=False, with_wc=True)
    one_call = measure_decode(torch, pkg, args, phases, matmuls=True, with_wc=False, by_phase=False)
    decode_m4 = measure_decode_m4(torch, pkg, args, phases)
    del layers, head, phases
    torch.cuda.empty_cache()
    gemm = None if args.no_gemm else measure_gemm(torch, pkg, args)
    ceilings = measure_ceilings(torch, pkg)
    # one llama.cpp block type (Q4_K, the type the reference's GPU path keeps) at the 8B MLP's shapes, decode and a
    # prompt of 512 tokens (--configs: every type)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(12)
    blocks_q4k = measure_blocks(torch, pkg, args, gen, names=("Q4_K",), prompts=(512,))
    torch.cuda.empty_cache()
    configs = None if args.no_configs else measure_configs(torch, pkg, args, extras=args.configs)
    cpu = None if args.no_cpu else cpu_baseline(args)
    headline = one_call if args.mode == "matmuls" else separate
    achieved = separate["gemv_GBps"]
    line = {
        "metric": METRIC, "value": round(headline["GBps"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(headline["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic (seeded, generated on the GPU)",
        "config": {"workload": "Llama-3-8B Q8 decode GEMV, M=1: 32 layers x (q/k/v, o, gate/up, down) + lm-head "
                               "[128256, 4096]; a phase is quantize_x + matmul_q8r of its matrices (BASELINE "
                               "configs[3])", "mode": args.mode,
                   "step_bytes": headline["step_bytes"], "parallelism": "1 GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_per_launch(),
                     "kernel": "gemv_relaxed<8,1,false,0,32,…> (32 lanes a row; chunks of 4 steps, of 2 for the down projection)",
                     "avg_launch_us": round(separate["gemv_avg_launch_us"], 3),
                     "bytes_per_launch": round(separate["gemv_bytes_per_launch"])},
        "cpu_baseline": cpu,
        "detail": {"quantize_then_phase": separate, "quantize_then_phase_with_wc": separate_wc,
                   "hq_matmuls": one_call, "decode_m4": decode_m4,
                   "prefill_gemm": gemm, "ceilings": ceilings, "blocks_q4k": blocks_q4k, "configs": configs},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
