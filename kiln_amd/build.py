"""Build libkiln_hip.so (gfx950) in-tree with hipcc.

    python -m kiln_amd.build          # compile every source, link the library

Each .hip source under kiln_amd/csrc is compiled to an object in parallel,
then linked into kiln_amd/libkiln_hip.so. Packed-FP32 VALU instructions are
disabled for device code (-packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")
RUNNER_SRC = os.path.join(os.path.dirname(HERE), "tests", "cpp", "kiln_host_run.cpp")
RUNNER = os.path.join(HERE, "kiln_host_run")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkiln_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: str, build_dir: str = BUILD, extra=()) -> str:
    obj = os.path.join(build_dir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *CFLAGS, *extra, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, out: str = LIB, extra=(), build_dir: str = BUILD) -> str:
    """Compile and link; `extra` adds hipcc flags, `out`/`build_dir` redirect
    the library and objects (used to build tuning variants side by side)."""
    os.makedirs(build_dir, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip"))) + sorted(glob.glob(os.path.join(HOST, "*.cpp")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, build_dir, extra), srcs))
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    # A kernel template whose host-side stub was not emitted links into a
    # shared library without complaint; refuse such a library here.
    nm = subprocess.run(["nm", "-C", "--undefined-only", tmp], capture_output=True, text=True)
    missing = [l for l in nm.stdout.splitlines() if "__device_stub__" in l]
    if missing:
        raise RuntimeError("kernel launch stubs missing from the library:\n" + "\n".join(missing[:10]))
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    if out == LIB:
        if os.path.exists(RUNNER_SRC):
            build_runner(verbose)
        build_probes(verbose)
    return out


def build_probes(verbose: bool = False) -> str:
    """The hardware-ceiling probes (kiln_amd/probes), a library of their own."""
    src = os.path.join(HERE, "probes", "kh_probes.hip")
    out = os.path.join(HERE, "probes", "libkh_probes.so")
    cmd = [HIPCC, *CFLAGS, "-shared", src, "-o", out + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building the probes failed:\n{r.stdout}\n{r.stderr}")
    os.replace(out + ".tmp", out)
    if verbose:
        print(f"built {out}")
    return out


def build_runner(verbose: bool = False) -> str:
    """The C++ host-layer test driver, linked against libkiln_hip.so."""
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", RUNNER_SRC, "-o", RUNNER + ".tmp", f"-L{HERE}", "-lkiln_hip",
           "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building the host test driver failed:\n{r.stdout}\n{r.stderr}")
    os.replace(RUNNER + ".tmp", RUNNER)
    if verbose:
        print(f"built {RUNNER}")
    return RUNNER


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
