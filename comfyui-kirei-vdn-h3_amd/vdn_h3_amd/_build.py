"""Build ``libvdnh3.so`` for gfx950 with hipcc (in-tree, no JIT cache).

Usage: ``python -m vdn_h3_amd._build`` (from ``comfyui-kirei-vdn-h3_amd/``) or
``__graft_entry__.build()`` at the repository root. Every call recompiles.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
CSRC = ROOT / "csrc"
BUILD_DIR = ROOT / "_build"
LIB_PATH = PKG_DIR / "libvdnh3.so"
ARCH = os.environ.get("VDNH3_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU forms (v_pk_*_f32) are disabled for every device pass: hipcc would
# otherwise generate them from ordinary float code, and some of their forms have given
# silently wrong results on MI355X.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__"]
# Per-source additions (none at present). Every source keeps IEEE NaN semantics: the window
# attention file also normalises raw q / k, whose non-finite values must propagate as they do in
# the standalone q / k pass (the fmaxf row reductions cost three canonicalising v_max per tile).
EXTRA_FLAGS: dict[str, list[str]] = {}


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libvdnh3.so")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [_hipcc(), *HIP_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    else:
        cmd = [_hipcc(), *CXX_FLAGS, "-I/opt/rocm/include", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source under ``csrc/`` and link ``vdn_h3_amd/libvdnh3.so``."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
