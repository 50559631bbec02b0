"""Build libkrq.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python kernel-rush-qwen_amd/build_lib.py

One hipcc -c per source (run in parallel), then one hipcc -shared link. Objects go to
kernel-rush-qwen_amd/_build/, the library to kernel-rush-qwen_amd/kernels/libkrq.so.

    python kernel-rush-qwen_amd/build_lib.py --timeline

builds the same sources with -DKRQ_TIMELINE (per-block wall-clock stamps in the FP8 GEMV, read by
timeline.py) into kernels/libkrq_timeline.so; the shipped library never carries them.
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "kernels", "libkrq.so")
TIMELINE_OUT = os.path.join(HERE, "kernels", "libkrq_timeline.so")
SOURCES = ["quant.hip", "gemv_fp8.hip", "gemv_bf16.hip", "lmhead.hip", "mlp.hip", "fused_gemv.hip", "fused_fp8.hip", "gemm_fp8.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in the generated code.
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build(verbose=False, timeline=False):
    build_dir = os.path.join(BUILD, "timeline") if timeline else BUILD
    out = TIMELINE_OUT if timeline else OUT
    flags = FLAGS + (["-DKRQ_TIMELINE"] if timeline else [])
    os.makedirs(build_dir, exist_ok=True)
    objs = [os.path.join(build_dir, src.replace(".hip", ".o")) for src in SOURCES]

    def compile_one(src, obj):
        cmd = [HIPCC, *flags, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)

    workers = max(1, min(len(SOURCES), os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(compile_one, SOURCES, objs))  # re-raises the first failure
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, timeline="--timeline" in sys.argv))
