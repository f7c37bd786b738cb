"""Compile the gfx950 attention library in-tree: mugen_amd/libmugen_attn.so.

hipcc cross-compiles for gfx950 without a GPU.  Each .hip source is
compiled to an object in parallel, then linked into one shared library
that exports the C ABI declared in include/mugen_attn.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libmugen_attn.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["capi.hip", "engine.hip", "gqa_decode.hip", "gqa_prefill.hip", "kv_q4.hip", "mla_cache.hip",
           "mla_decode.hip", "mla_proj.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build mugen_amd)")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-I", INCLUDE, "-I", CSRC,
        # no packed fp32 VALU ops (v_pk_*_f32) in device code: some of their
        # forms have produced silently wrong results on this hardware
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
    ]


def _compile(src: str, obj_dir: str) -> str:
    obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *common_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    obj_dir = os.path.join(HERE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    build_selftest(verbose)
    return LIB_PATH


SELFTEST = os.path.join(HERE, "engine_selftest")


def build_program(src: str, exe: str, verbose: bool = False) -> str:
    """A host program over the provider header (include/mugen_attn_engine.hpp),
    linked against the in-tree library (rpath relative to the program)."""
    tmp = exe + ".tmp"
    rel = os.path.relpath(HERE, os.path.dirname(os.path.abspath(exe)))
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++20", "-I", INCLUDE, src, "-o", tmp,
           "-L", HERE, "-lmugen_attn", "-Wl,-rpath,$ORIGIN/" + rel, "-Wno-unused-command-line-argument"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{os.path.basename(src)} build failed:\n{r.stderr}")
    os.replace(tmp, exe)
    if verbose:
        print(f"built {exe}")
    return exe


def build_selftest(verbose: bool = False) -> str:
    """The C++ provider check (engine_selftest.cpp, run by the GPU tests)."""
    return build_program(os.path.join(HERE, "engine_selftest.cpp"), SELFTEST, verbose)


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
