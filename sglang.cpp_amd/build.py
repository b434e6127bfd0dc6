"""Build the gfx950 attention library (libsgl_attn.so) in-tree.

Each HIP source under csrc/ is compiled for gfx950 with hipcc and linked
into one shared library next to this file; the C++ backend extension
(LibTorch host code over the C ABI) is built by build_backend().
Run directly: python sglang.cpp_amd/build.py
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libsgl_attn.so"
LIB_PATH = PKG_DIR / LIB_NAME

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-fp32 VALU ops are disabled for all device code (see the toolchain
# notes in DESIGN.md); hipcc's host pass warns that it does not know the
# feature, which is harmless.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
]

SOURCES = ["kv_store.hip", "metadata.hip", "rope_norm.hip", "decode.hip", "prefill.hip"]


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # Surface real diagnostics, drop the known host-pass feature warning.
    lines = [ln for ln in res.stderr.splitlines()
             if "packed-fp32-ops" not in ln and "warning: unknown" not in ln and ln.strip()]
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")


def build_lib(jobs: int = 8) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = []
        for name in SOURCES:
            src = CSRC / name
            obj = BUILD_DIR / (name + ".o")
            objs.append(obj)
            futs.append(ex.submit(_compile, src, obj))
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build(jobs: int = 8) -> None:
    build_lib(jobs)


if __name__ == "__main__":
    build()
    print(LIB_PATH)
