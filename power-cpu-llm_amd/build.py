"""Build recipe of the gfx950 attention library (libpcl_attention.so).

Run as a script or call build(). hipcc cross-compiles for gfx950 without a
GPU; the shared library lands next to this file, where the Python loader,
the tests and bench.py look for it.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libpcl_attention.so")
OBJ_DIR = os.path.join(HERE, "_build")
SOURCES = ["csrc/split_kv.hip", "csrc/pipe_kv.hip", "csrc/spread_kv.hip",
           "csrc/tiled.hip", "csrc/tiled_wide.hip", "csrc/fan_kv.hip",
           "csrc/api.hip", "csrc/kv_cache.hip", "csrc/head_transform.hip",
           "csrc/output_block.hip"]
HEADERS = ["csrc/attention_device.hpp", "csrc/context.hpp", os.path.join(ROOT, "include", "pcl_attention.h")]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # No contraction: every multiply-add the kernels mean to fuse is written
    # as an explicit fma, so all kernels share one operation sequence.
    "-ffp-contract=off",
    # No packed fp32 instructions in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-I" + os.path.join(ROOT, "include"),
]


def _run(cmd, verbose):
    res = subprocess.run(cmd, cwd=HERE, capture_output=True, text=True)
    noise = "packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        sys.stderr.write(err + "\n")
        raise subprocess.CalledProcessError(res.returncode, cmd, res.stdout, res.stderr)
    if verbose and err.strip():
        sys.stderr.write(err + "\n")


def build(verbose=False):
    """Compile every source (one hipcc process per file, in parallel) and
    link them into LIB; raises CalledProcessError on failure."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(OBJ_DIR, exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objs = [os.path.join(OBJ_DIR, os.path.basename(s) + ".o") for s in SOURCES]
    cmds = [[HIPCC] + compile_flags + ["-c", "-o", o, os.path.join(HERE, s)]
            for s, o in zip(SOURCES, objs)]
    jobs = max(1, min(len(cmds), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(jobs) as pool:
        for f in [pool.submit(_run, c, verbose) for c in cmds]:
            f.result()
    _run([HIPCC] + FLAGS + ["-o", LIB] + objs, verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
