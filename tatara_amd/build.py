"""Builds the gfx950 HIP library tatara_amd/libtatara_hip.so in-tree.

Every source under tatara_amd/csrc is compiled by hipcc for gfx950 only,
with fp contraction off (the kernels reproduce the reference CPU arithmetic
operation for operation) and without packed-FP32 instructions.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtatara_hip.so"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, "-c", *FLAGS, str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def source_digest() -> str:
    """A short SHA-256 over the kernel sources (every csrc file and the C
    header, by name and content): it names the kernels a measurement was
    taken with where no git metadata travels with the tree."""
    import hashlib

    h = hashlib.sha256()
    files = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.hpp")) + [PKG.parent / "include" / "tatara_hip.h"])
    for f in files:
        h.update(f.name.encode() + b"\0")
        h.update(f.read_bytes())
    return h.hexdigest()[:12]


def build(jobs: int | None = None) -> Path:
    """Compiles every source and links the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_code_object(src: Path, out: Path | None = None) -> Path:
    """Compiles one HIP source into a gfx950 code object (hipcc --genco) for
    tatara_module_load_image; returns its path (default: src with .hsaco)."""
    src = Path(src)
    out = Path(out) if out else src.with_suffix(".hsaco")
    tmp = out.with_suffix(out.suffix + ".tmp")
    cmd = [HIPCC, "--genco", *FLAGS, str(src), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc --genco failed for {src.name}:\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())
    sys.exit(0)
