"""Build libhexanima_hip.so for MI355X (gfx950) with hipcc, in-tree (hexanima_amd/libhexanima_hip.so).

Each .hip source is compiled to an object under hexanima_amd/_build/ (in parallel), then linked into one shared
library exporting the C-ABI of include/hexanima_hip.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libhexanima_hip.so")
# the MOSS build of the block interface: exports the reference's mega_block name with the MOSS semantics
MOSS_LIB = os.path.join(HERE, "libhexanima_moss.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
PROGRAMS = ["hxa_run", "hxa_blk"]
SOURCES = ["gemm.hip", "attention.hip", "elementwise.hip", "runtime.hip", "dit.hip", "noalloc.hip"]

ARCH = os.environ.get("HXA_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
# packed-fp32 instructions are disabled in device code: ordinary scalar / float2 code only
CFLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
          "-Wno-pass-failed", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, src.replace(".hip", ".o"))
    cmd = [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        msg = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    return obj


def _stale(src: str) -> bool:
    obj = os.path.join(OBJ, src.replace(".hip", ".o"))
    if not os.path.exists(obj):
        return True
    deps = [os.path.join(CSRC, src)] + [os.path.join(CSRC, h) for h in os.listdir(CSRC) if h.endswith(".h")]
    deps.append(os.path.join(os.path.dirname(HERE), "include", "hexanima_hip.h"))
    return max(os.path.getmtime(d) for d in deps) > os.path.getmtime(obj)


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compile every HIP source (incremental: only those newer than their object) and link the shared library;
    returns its path."""
    os.makedirs(OBJ, exist_ok=True)
    todo = [s for s in SOURCES if _stale(s)] if incremental else SOURCES
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        list(ex.map(_compile, todo))
    objs = [os.path.join(OBJ, s.replace(".hip", ".o")) for s in SOURCES]
    tmp = LIB + ".tmp"
    # -Bsymbolic-functions: the library's own calls bind to its own definitions, also when libhexanima_moss.so's
    # mega_block is loaded first in a process
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-Bsymbolic-functions", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    tmp = MOSS_LIB + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-I", INCLUDE, "-o", tmp,
           os.path.join(CSRC, "moss_abi.cpp"), "-L", HERE, "-lhexanima_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"libhexanima_moss.so failed:\n{r.stderr}")
    os.replace(tmp, MOSS_LIB)
    # the host programs above the block interface: the megarun-protocol runner and the blk_main-style harness
    for prog in PROGRAMS:
        out = os.path.join(HERE, prog)
        cmd = ["g++", "-O2", "-std=c++17", "-Wall", "-I", INCLUDE, "-o", out + ".tmp", os.path.join(CSRC, prog + ".cpp"),
               "-L", HERE, "-lhexanima_hip", "-Wl,-rpath,$ORIGIN"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"{prog} failed:\n{r.stderr}")
        os.replace(out + ".tmp", out)
    if verbose:
        print("built", LIB)
    return LIB


SAN_DIR = os.path.join(HERE, "_san")


def build_sanitized(verbose: bool = False) -> str:
    """The host programs (hxa_run, hxa_blk) built with AddressSanitizer + UndefinedBehaviorSanitizer into
    hexanima_amd/_san/, linking the ordinary libhexanima_hip.so (host code only: no device code is instrumented).
    Run the runner tests on them with HXA_PROG_DIR=hexanima_amd/_san."""
    os.makedirs(SAN_DIR, exist_ok=True)
    for prog in PROGRAMS:
        out = os.path.join(SAN_DIR, prog)
        cmd = ["g++", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
               "-std=c++17", "-Wall", "-I", INCLUDE, "-o", out + ".tmp", os.path.join(CSRC, prog + ".cpp"), "-L", HERE,
               "-lhexanima_hip", "-Wl,-rpath,$ORIGIN/.."]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"{prog} (sanitized) failed:\n{r.stderr}")
        os.replace(out + ".tmp", out)
    if verbose:
        print("built", SAN_DIR)
    return SAN_DIR


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        build_sanitized(verbose=True)
    else:
        build(verbose=True, incremental="--incremental" in sys.argv)
    sys.exit(0)
