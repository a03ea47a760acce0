"""Build libdlmk.so (HIP kernels for gfx950 + host bookkeeping) in-tree.

The library is compiled directly with hipcc -- no torch extension machinery --
so its C ABI (include/dlmk.h) carries no torch types and can be linked from
C, C++, Rust (build.rs) or loaded through ctypes.

    python -m dlm_amd.build          # compile dlm_amd/libdlmk.so
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD_DIR = os.path.join(PKG, "_build")
LIB_PATH = os.path.join(PKG, "libdlmk.so")

ARCH = "gfx950"
SOURCES = ["runtime.hip", "kv_cache.cpp", "kv_append.hip", "attention.hip", "attention_f32.hip",
           "attention_f16.hip", "attention_bf16.hip", "attention_i8.hip", "attention_i4.hip",
           "blocks.hip",
           "decode_block.hip"]

# -packed-fp32-ops: keep the compiler from emitting packed FP32 VALU ops.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _compile(src: str, build_dir: str = BUILD_DIR, defines=()) -> str:
    obj = os.path.join(build_dir, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *(f"-D{d}" for d in defines), f"-I{INCLUDE}", f"-I{CSRC}", "-c",
           os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compiling {src} failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, out: str = LIB_PATH, defines=()) -> str:
    """Compile every source and link libdlmk.so (dlm_amd/libdlmk.so unless `out`
    names another path; `defines` are extra -D macros); returns its path."""
    build_dir = BUILD_DIR if out == LIB_PATH else out + ".objs"
    os.makedirs(build_dir, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile(s, build_dir, defines), SOURCES))
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"linking libdlmk.so failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
