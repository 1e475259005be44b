"""Build recipe for the gfx950 C-ABI library ``aila_amd/libaila_hip.so``.

Every source under ``aila_amd/csrc`` (``*.hip`` device code, ``*.cpp`` host
code) is compiled by hipcc for gfx950 into ``aila_amd/_build`` and linked
into one shared library. The C++ ``ops::`` layer (``aila_amd/host``) links
against it as ``libaila_ops.so``; ``aila_amd/probe`` builds the benchmark's
streaming-read probe into ``libaila_probe.so``, which the product never
loads. Run ``python -m aila_amd.build``.

HIP code is compiled with packed-FP32 instruction selection disabled
(``-packed-fp32-ops``); hipcc's host pass warns that it does not know that
target feature, which is harmless.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libaila_hip.so")
OPS_LIB = os.path.join(HERE, "libaila_ops.so")
PROBE_LIB = os.path.join(HERE, "libaila_probe.so")
HOST = os.path.join(HERE, "host")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    jobs = min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", LIB, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    # Load check: a kernel template whose host-side launch stub was not
    # emitted leaves an undefined symbol that only shows at dlopen.
    r = subprocess.run([sys.executable, "-c", f"import ctypes; ctypes.CDLL({LIB!r})"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{LIB} does not load:\n{r.stderr.strip().splitlines()[-1]}")
    # C++ ops:: layer over the C ABI (host code only)
    host_srcs = sorted(glob.glob(os.path.join(HOST, "*.cpp")))
    cmd = [HIPCC, "-std=c++17", "-O2", "-fPIC", "-shared", "-I", HOST, "-I", os.path.join(ROOT, "include"),
           *host_srcs, "-o", OPS_LIB, "-L", HERE, "-laila_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"ops layer build failed:\n{r.stderr}")
    # measurement probe for the benchmark (not part of the product library)
    cmd = [HIPCC, *COMMON, "-shared", os.path.join(HERE, "probe", "stream_read.hip"), "-o", PROBE_LIB]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"probe build failed:\n{r.stderr}")
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources, {OPS_LIB} and {PROBE_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
