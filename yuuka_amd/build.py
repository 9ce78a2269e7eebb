"""Builds libyuuka_hip.so (gfx950) in-tree with hipcc.

Every source under yuuka_amd/csrc is compiled to an object in
yuuka_amd/_build and linked into yuuka_amd/lib/libyuuka_hip.so. Packed FP32
instruction selection is disabled on every HIP compile.
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
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libyuuka_hip.so"

ARCH = "gfx950"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CFLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Wall",
    "-Wno-unused-function",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the GEMM epilogues read every result lane once.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def sources() -> list[Path]:
    return sorted(p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp"))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [HIPCC, *CFLAGS, "-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, len(srcs))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


def build_oracle(verbose: bool = False) -> Path:
    """Compiles the CPU restatement (test infrastructure) with its Makefile."""
    oracle = PKG.parent / "oracle"
    r = subprocess.run(["make", "-C", str(oracle), "-s", "-B"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {oracle / 'liboracle.so'}")
    return oracle / "liboracle.so"


def _stale(target: Path, srcs) -> bool:
    if not target.exists():
        return True
    t = target.stat().st_mtime
    return any(p.stat().st_mtime > t for p in srcs)


def ensure_built() -> None:
    """Builds the library (and the oracle) when missing or older than any of
    its sources, so that a stale build never runs silently."""
    hdr = PKG.parent / "include"
    if _stale(LIB, [*sources(), *CSRC.glob("*.h"), *hdr.glob("*.h")]):
        build()
    oracle = PKG.parent / "oracle"
    if _stale(oracle / "liboracle.so", [*oracle.glob("*.c"), *oracle.glob("*.h"), oracle / "Makefile"]):
        build_oracle()


if __name__ == "__main__":
    build(verbose=True)
    if "--no-oracle" not in sys.argv:
        build_oracle(verbose=True)
