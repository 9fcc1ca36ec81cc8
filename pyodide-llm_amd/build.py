"""Builds libhq.so (the HIP kernels and their C-ABI, include/hq.h) in-tree for gfx950 with hipcc.

    python pyodide-llm_amd/build.py [--jobs N]

Every source is compiled again on every call.  Flags: -ffp-contract=off (every float operation written in the
kernels is one IEEE operation, as the reference's are), denormals kept, and packed FP32 instructions off.  The build
fails if a kernel spills registers to scratch memory (the compiler's resource-usage remarks say so).
"""
import argparse
import concurrent.futures
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJ = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libhq.so")
SOURCES = ["quantize.hip", "gemv.hip", "gemm.hip", "gemm_tol.hip", "blocks.hip", "columns.hip", "ceilings.hip", "abi.cpp"]
# blocks.hip's prompt tile keeps its matrix-core results in ordinary VGPRs (no copies out of AGPRs: it has registers
# to spare and reads every result on the VALU)
EXTRA = {"blocks.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         # the token kernels' scalar arguments (one job's fields) in the waves' scalar registers at launch
         "gemv.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
         # quantize_x's arguments likewise (14 dwords): it runs before every phase of a decode step
         "quantize.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", CSRC, "-I", INCLUDE,
]


REMARK = re.compile(r"remark: +(Function Name|ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill): (\S+)")


def _spills(stderr):
    """the kernels the resource-usage remarks report spilling or using scratch memory"""
    bad, name = [], None
    for m in REMARK.finditer(stderr):
        if m.group(1) == "Function Name":
            name = m.group(2)
        elif int(m.group(2)) > 0 and (not bad or bad[-1] != name):
            bad.append(name)
    return bad


def _compile(src):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-Rpass-analysis=kernel-resource-usage", "-x", "hip", "-c",
           os.path.join(CSRC, src), "-o", obj]
    run = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so: harmless
    noise = "is not a recognized feature for this target"
    lines = run.stderr.splitlines()
    # the remarks (and the source lines and carets they quote) are read, not shown
    keep, skip = [], 0
    for line in lines:
        if "[-Rpass-analysis=kernel-resource-usage]" in line:
            skip = 2 if "Function Name" in line else 0
            continue
        if skip:
            skip -= 1
            continue
        if noise not in line:
            keep.append(line)
    err = "\n".join(keep)
    if run.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    bad = _spills(run.stderr)
    if bad:
        raise RuntimeError(f"{src}: kernels spill registers to scratch memory: {', '.join(bad)}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(jobs=None):
    """Compile every source and link libhq.so; returns its path."""
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(_compile, SOURCES))
    tmp = LIBRARY + ".tmp"
    run = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objects],
                         capture_output=True, text=True)
    if run.returncode != 0:
        raise RuntimeError(f"link failed:\n{run.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--jobs", type=int, default=None)
    print(build(parser.parse_args().jobs))
