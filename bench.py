"""bench.py — the hot path's headline numbers on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-gemm]

A step is one decode token of the Llama-3-8B-shaped Q8 path: per layer the reference's
four phases (src/runtime/forward/attention.ts:173, ffn.ts:27-30): quantize_x of the input, then q / k / v
(4096, 1024, 1024 rows x 4096) in one phase, o (4096 x 4096), gate and up (2 x 14336 x 4096) in one phase, down
(4096 x 14336); 32 layers, then the classifier (128256 x 4096).  Every layer has its own weights (8.44 GB in all, far
past the 256 MB Infinity Cache), int8 uniform in [-127, 127] with |N(0, 0.02)| / 127 scales, activations N(0, 1):
synthetic, generated on the GPU from a seed.  The products are matmul_q8r's (relaxed form, quantize_x bias 64); each
phase is one hq_matmuls() call (the reference's matmulsAlike: quantize_x inside the products' launch), the
corrections derived in the kernel (wc = NULL: the same integers as int8_sums' wc, and 12.5 % fewer bytes).  Beside it:
the same step as quantize_x then hq_phase(), without and with the caller's wc.

value: algorithmic bytes of a step (1.125 B a weight, the activations' bytes and scales, 4 B an output; jobs.ts:448-450)
over the step's time, with all inputs resident in HBM.  The step runs as a HIP graph of its launches (captured once).
roofline: the GEMV kernel alone, from HIP events around every phase launch of an eager pass of the same steps.
Also reported: the int8 prefill GEMM (config 3's M = 2048 over one layer's matrices) in TOPS against the dense int8
MFMA peak, and the oracle (the C restatement, oracle/) on the host's cores as the CPU baseline.
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
        bytes_ = sum(m.bytes() + a.bytes() + 4 * m.rows for m, _ in mats)
        tables.append((a, table, len(entries), bytes_))
    return tables


def run_step(lib, tables, stream, fused, events=None):
    for i, (a, table, njobs, _) in enumerate(tables):
        if fused:  # engine.ts's matmulsAlike: quantize_x inside the products' launch
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


def measure_decode(torch, pkg, args, phases, fused, with_wc):
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
            run_step(lib, tables, handle, fused)
        pkg.check(lib.hq_last_error())
        torch.cuda.synchronize()
        # the timed region: K steps as a HIP graph of one step's launches
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            run_step(lib, tables, handle, fused)
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            g.replay()
        torch.cuda.synchronize()
        graph_s = (time.perf_counter() - t0) / args.steps
        # the same K steps launched one by one, HIP events around every products launch: the GEMV kernel's times
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in tables]
        gemv_ms, launches = 0.0, 0
        kinds = {}
        t0 = time.perf_counter()
        for step in range(args.steps):
            run_step(lib, tables, handle, fused, events)
            torch.cuda.synchronize()
            for i, ((e0, e1), t) in enumerate(zip(events, tables)):
                ms = e0.elapsed_time(e1)
                gemv_ms += ms
                launches += 1
                name = ["qkv", "o", "gate_up", "down"][i % 4] if i < 4 * LAYERS else "lm_head"
                k = kinds.setdefault(name, [0.0, 0.0, 0])
                k[0] += ms
                k[1] += t[3]
                k[2] += 1
        pkg.check(lib.hq_set_stream(None))
    out["ms_per_step"] = 1e3 * graph_s
    out["GBps"] = step_bytes / graph_s / 1e9
    out["gemv_avg_launch_us"] = 1e3 * gemv_ms / launches
    out["gemv_bytes_per_launch"] = step_bytes / len(tables)
    out["gemv_GBps"] = step_bytes * args.steps / (gemv_ms * 1e-3) / 1e9
    out["phases"] = {n: {"us": round(1e3 * v[0] / v[2], 2), "GBps": round(v[1] / (v[0] * 1e-3) / 1e9, 1)}
                     for n, v in kinds.items()}
    return out


def measure_gemm(torch, pkg, args):
    """config 3's prefill: M = 2048 tokens through one layer's matrices (q, k, v, o, gate, up, down)."""
    lib = pkg.library()
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(5)
    M = 2048
    shapes = [(4096, HIDDEN), (1024, HIDDEN), (1024, HIDDEN), (HIDDEN, HIDDEN), (FFN, HIDDEN), (FFN, HIDDEN),
              (HIDDEN, FFN)]
    mats = [Matrix(torch, gen, r, n) for r, n in shapes]
    acts = {}
    for n in (HIDDEN, FFN):
        x = torch.randn(M, n, device="cuda:0", generator=gen)
        frame = n + 4 * (n // 32)
        buf = torch.empty(M * frame, dtype=torch.uint8, device="cuda:0")
        pkg.check(lib.hq_quantize_x_batch(buf.data_ptr(), buf.data_ptr() + n, x.data_ptr(), n, 64, M, frame, 4 * n, None))
        acts[n] = (buf, frame)
    outs = [torch.empty(M, r, dtype=torch.float32, device="cuda:0") for r, _ in shapes]

    def run():
        for m, o in zip(mats, outs):
            buf, frame = acts[m.n]
            lib.hq_matmul_q8r_tile_ex(o.data_ptr(), buf.data_ptr(), buf.data_ptr() + m.n, m.w.data_ptr(),
                                      m.ws.data_ptr(), None, m.n, 0, m.rows, M, 4 * m.rows, frame, None)

    run()
    pkg.check(lib.hq_last_error())
    torch.cuda.synchronize()
    reps = max(2, args.steps // 5)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    s = e0.elapsed_time(e1) * 1e-3 / reps
    ops = sum(2.0 * M * r * n for r, n in shapes)
    return {"M": M, "tops": ops / s / 1e12, "frac": ops / s / 1e12 / INT8_PEAK_TOPS, "ms_per_layer": s * 1e3}


def cpu_baseline(args):
    """The oracle's matmul_q8r (oracle/oracle.c: the reference arithmetic in C, scalar) on the host's cores, rows cut
    as the reference's phase() cuts them, over one 8B layer's matrices (~245 MB, past the host's caches)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    threads = min(16, os.cpu_count() or 1)
    rng = np.random.default_rng(9)
    shapes = [(4096, HIDDEN), (1024, HIDDEN), (1024, HIDDEN), (HIDDEN, HIDDEN), (FFN, HIDDEN), (FFN, HIDDEN),
              (HIDDEN, FFN)]
    total_s, total_bytes = 0.0, 0.0
    for rows, n in shapes:
        w = rng.integers(-127, 128, rows * n, dtype=np.int8)
        ws = (np.abs(rng.standard_normal(rows * n // 32)) * 0.02 / 127).astype(np.float32)
        wc = oracle.int8_sums(w)
        xq, xs = oracle.quantize_x(rng.standard_normal(n).astype(np.float32), 64)
        s = oracle.time_gemv("matmul_q8r", xq, xs, w, ws, wc, n, rows, threads, 3)
        total_s += s
        total_bytes += rows * n * 1.125 + n * 1.125 + 4 * rows
    return {"value": total_bytes / total_s / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": "oracle matmul_q8r (C restatement, scalar) over one Llama-3-8B layer's 7 matrices at M=1, "
                      f"{threads} threads, fastest of 3 runs each"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--mode", choices=("phase", "fused"), default="phase",
                    help="the headline's phases: quantize_x then hq_phase (the reference's ready() + phase()), or "
                         "hq_matmuls (quantize_x inside the products' launch)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the path is built for one MI355X (rows would shard across GPUs with an "
              "all-gather of the outputs, which this build does not run); use --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    pkg = load_package()
    torch.cuda.set_device(0)
    pkg.check(pkg.library().hq_init())
    from pyodide_llm_amd import jobs
    layers, head, phases = build_decode(torch, jobs, pkg.library())
    fused = measure_decode(torch, pkg, args, phases, fused=True, with_wc=False)
    separate = measure_decode(torch, pkg, args, phases, fused=False, with_wc=False)
    separate_wc = measure_decode(torch, pkg, args, phases, fused=False, with_wc=True)
    del layers, head, phases
    torch.cuda.empty_cache()
    gemm = None if args.no_gemm else measure_gemm(torch, pkg, args)
    cpu = None if args.no_cpu else cpu_baseline(args)
    derived = fused if args.mode == "fused" else separate
    achieved = derived["gemv_GBps"]
    line = {
        "metric": METRIC, "value": round(derived["GBps"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(derived["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic (seeded, generated on the GPU)",
        "config": {"workload": "Llama-3-8B Q8 decode GEMV, M=1: 32 layers x (q/k/v, o, gate/up, down) + lm-head "
                               "[128256, 4096]; a phase is quantize_x + matmul_q8r of its matrices (BASELINE "
                               "configs[3])", "mode": args.mode,
                   "step_bytes": derived["step_bytes"], "parallelism": "1 GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv_relaxed<8,1,false,FUSED>" if args.mode == "fused" else "gemv_relaxed<8,1,false,GLOBAL>",
                     "avg_launch_us": round(derived["gemv_avg_launch_us"], 3),
                     "bytes_per_launch": round(derived["gemv_bytes_per_launch"])},
        "cpu_baseline": cpu,
        "detail": {"fused": fused, "quantize_then_phase": separate, "quantize_then_phase_with_wc": separate_wc,
                   "prefill_gemm": gemm},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
